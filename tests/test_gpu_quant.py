"""int8 absmax quantisation and dequantisation on the GPU vs the oracle:
codes, scales and fp16 outputs bit-exact (round half to even, IEEE division)."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(11))


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def all_fp16_rows(cols=496):
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    allv = np.concatenate([h, h | 0x8000])
    n = (allv.size // cols) * cols
    return RNG.permutation(allv[:n]).reshape(-1, cols)


def run_rows(lib, x):
    rows, cols = x.shape
    xb, qb, sb = dev(x), empty(x.size), empty(4 * rows)
    ok(lib.cuda_quantize_weights_per_row(qb.vp, sb.vp, xb.vp, rows, cols), "quant rows")
    return get(qb, np.int8, x.shape), get(sb, np.float32, (rows,))


@pytest.mark.parametrize("cols", [496, 4096, 14336, 1000, 65536, 70000])
def test_per_row_quant_bit_exact(lib, ora, cols):
    banner(f"per-row quant cols={cols}")
    if cols == 496:
        x = all_fp16_rows(cols)
    else:
        x = f16(RNG.standard_t(3, (37, cols)) * RNG.uniform(0.01, 100, (37, 1)))
    q, s = run_rows(lib, x)
    qw, sw = ora.quant_rows(x)
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")


def test_per_row_quant_zero_rows_and_ties(lib, ora):
    banner("per-row quant zero rows and ties")
    x = np.zeros((4, 256), np.uint16)
    x[1, 0] = f16(127.0)[()]            # scale 1: codes are rint of the values
    x[1, 1:9] = f16([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5])
    x[2, :] = f16(RNG.standard_normal(256))
    q, s = run_rows(lib, x)
    qw, sw = ora.quant_rows(x)
    assert_bits_equal(q, qw, "codes")
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert (q[0] == 0).all() and s[0] == 1.0
    assert q[1, 1:9].tolist() == [0, 2, 2, 0, -2, -2, 126, -126]


@pytest.mark.parametrize("cols", [4096, 1000])
def test_per_row_quant_rows_with_infinities(lib, ora, cols):
    """A row holding +-inf has scale inf; its finite values get code 0 (v / inf = 0),
    as in the oracle. Codes of the infinite elements themselves are unspecified."""
    banner(f"per-row quant rows with infinities cols={cols}")
    x = f16(RNG.standard_normal((6, cols)))
    x[1, 5] = 0x7C00          # +inf
    x[3, cols - 1] = 0xFC00   # -inf
    x[4, 0], x[4, 7] = 0x7C00, 0xFC00
    q, s = run_rows(lib, x)
    qw, sw = ora.quant_rows(x)
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert np.isinf(s[[1, 3, 4]]).all()
    finite = (x & 0x7C00) != 0x7C00
    assert_bits_equal(q[finite], qw[finite], "codes of finite elements")
    assert (q[[1, 3, 4]][finite[[1, 3, 4]]] == 0).all()


def run_norm_quant(lib, x, w, eps, residual=None):
    T, H = x.shape
    xb, wb, qb, sb = dev(x), dev(w), empty(x.size), empty(4 * T)
    if residual is None:
        ok(lib.ng_rmsnorm_quant_int8(qb.vp, sb.vp, xb.vp, wb.vp, T, H, C.c_float(eps)), "norm+quant")
        return get(qb, np.int8, x.shape), get(sb, np.float32, (T,))
    rb, rob = dev(residual), empty(x.nbytes)
    ok(lib.ng_add_rmsnorm_quant_int8(qb.vp, sb.vp, rob.vp, xb.vp, rb.vp, wb.vp, T, H, C.c_float(eps)),
       "add+norm+quant")
    return get(qb, np.int8, x.shape), get(sb, np.float32, (T,)), get(rob, np.uint16, x.shape)


@pytest.mark.parametrize("T,H", [(1, 4096), (64, 4096), (300, 5120), (8, 4100), (2, 65536)])
def test_rmsnorm_quant_bit_exact(lib, ora, T, H):
    banner(f"rmsnorm+int8 T={T} H={H}")
    x = f16(RNG.standard_t(3, (T, H)))
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    q, s = run_norm_quant(lib, x, w, 1e-5)
    qw, sw = ora.rmsnorm_quant(x, w, 1e-5)
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")


def test_rmsnorm_quant_matches_the_two_step_composition(lib, ora):
    """Fused kernel == cuda_rmsnorm followed by cuda_quantize_weights_per_row,
    both on the GPU (the composition it replaces)."""
    banner("rmsnorm+int8 vs composition")
    T, H = 128, 4096
    x = f16(RNG.standard_t(3, (T, H)) * 3)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    q, s = run_norm_quant(lib, x, w, 1e-5)
    xb, wb, yb = dev(x), dev(w), empty(x.nbytes)
    ok(lib.cuda_rmsnorm(yb.vp, xb.vp, wb.vp, T, H, C.c_float(1e-5)))
    q2b, s2b = empty(x.size), empty(4 * T)
    ok(lib.cuda_quantize_weights_per_row(q2b.vp, s2b.vp, yb.vp, T, H))
    assert_bits_equal(q, get(q2b, np.int8, (T, H)), "codes")
    assert_bits_equal(s, get(s2b, np.float32, (T,)), "scales")


@pytest.mark.parametrize("T,H", [(64, 4096), (9, 4100)])
def test_add_rmsnorm_quant_bit_exact(lib, ora, T, H):
    banner(f"add+rmsnorm+int8 T={T} H={H}")
    x = f16(RNG.standard_normal((T, H)))
    r = f16(RNG.standard_normal((T, H)) * 2)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    q, s, ro = run_norm_quant(lib, x, w, 1e-5, residual=r)
    qw, sw, row = ora.add_rmsnorm_quant(x, r, w, 1e-5)
    assert_bits_equal(ro, row, "residual_out")
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")


@pytest.mark.parametrize("n", [4096, 1 << 20, 12345, 7])
def test_per_tensor_quant_bit_exact(lib, ora, n):
    banner(f"per-tensor quant n={n}")
    x = f16(RNG.uniform(-1, 1, n) * RNG.choice([1, 30], n))
    xb, qb, sb = dev(x), empty(n), empty(4)
    ok(lib.cuda_quantize_per_tensor(qb.vp, sb.vp, xb.vp, n), "quant tensor")
    qw, sw = ora.quant_tensor(x)
    assert_bits_equal(get(sb, np.float32, (1,)).view(np.uint32), sw.view(np.uint32), "scale")
    assert_bits_equal(get(qb, np.int8, (n,)), qw, "codes")


@pytest.mark.parametrize("K,N", [(128, 64), (1000, 333), (4096, 4096), (3, 8)])
def test_per_column_quant_bit_exact(lib, ora, K, N):
    banner(f"per-column quant {K}x{N}")
    x = f16(RNG.standard_normal((K, N)) * RNG.uniform(0.01, 10, (1, N)))
    xb, qb, sb = dev(x), empty(x.size), empty(4 * N)
    ok(lib.cuda_quantize_weights(qb.vp, sb.vp, xb.vp, K, N), "quant cols")
    qw, sw = ora.quant_cols(x)
    assert_bits_equal(get(sb, np.float32, (N,)).view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(get(qb, np.int8, (K, N)), qw, "codes")


@pytest.mark.parametrize("rows,cols", [(256, 4096), (7, 100), (3, 16), (14336, 4096), (7, 1536), (1, 512), (5, 528)])
@pytest.mark.parametrize("per_row", [1, 0])
def test_dequant_weights_bit_exact(lib, ora, rows, cols, per_row):
    banner(f"dequant {rows}x{cols} per_row={per_row}")
    q = RNG.integers(-127, 128, (rows, cols)).astype(np.int8)
    n_sc = rows if per_row else cols
    sc = RNG.uniform(1e-3, 1e-2, n_sc).astype(np.float16).astype(np.float32)
    qb, sb, ob = dev(q), dev(sc), empty(2 * q.size)
    ok(lib.cuda_dequantize_weights(ob.vp, qb.vp, sb.vp, rows, cols, per_row), "dequant")
    want = ora.dequant(q, sc, "row" if per_row else "col")
    assert_bits_equal(get(ob, np.uint16, (rows, cols)), want, "dequant")


@pytest.mark.parametrize("n", [4096, 4099, 1 << 20, 512 * 7])
def test_dequant_per_tensor_bit_exact(lib, ora, n):
    banner(f"dequant per-tensor n={n}")
    q = RNG.integers(-128, 128, n).astype(np.int8)
    sc = np.float32([0.01])
    qb, sb, ob = dev(q), dev(sc), empty(2 * n)
    ok(lib.cuda_dequantize_per_tensor(ob.vp, qb.vp, sb.vp, n), "dequant tensor")
    assert_bits_equal(get(ob, np.uint16, (n,)), ora.dequant(q, sc, "tensor"), "dequant tensor")
