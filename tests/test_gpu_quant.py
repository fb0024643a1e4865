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


def nonfinite_rows(rows, cols):
    """Rows holding NaNs and infinities, the cases where the reference's rule
    (NaNs skipped by the fmaxf absmax, fmaxf(-127, fminf(127, q)) codes) differs
    from a naive maximum."""
    x = f16(RNG.standard_normal((rows, cols)) * RNG.uniform(0.1, 10, (rows, 1)))
    x[0, 3] = 0x7E00                           # a quiet NaN
    x[1, :] = 0x7E00                           # every element NaN: scale 1, codes +127
    x[2, 5], x[2, cols - 1] = 0x7C01, 0xFE00   # signalling and negative NaNs
    x[3, 7] = 0x7C00                           # +inf: scale inf, finite codes 0
    x[4, 0], x[4, 1] = 0xFC00, 0x7E00          # -inf and a NaN in one row
    x[5, cols // 2] = 0xFC00                   # -inf alone
    return x


@pytest.mark.parametrize("cols", [4096, 1000, 5120])
def test_per_row_quant_rows_with_nan_and_inf(lib, ora, cols):
    """Scales and every code bit-exact against the oracle, including the NaN and
    infinite elements (+127, as the reference's clamp order gives)."""
    banner(f"per-row quant rows with NaN and inf cols={cols}")
    x = nonfinite_rows(9, cols)
    q, s = run_rows(lib, x)
    qw, sw = ora.quant_rows(x)
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")
    assert np.isfinite(s[0]) and s[1] == 1 and np.isinf(s[[3, 4, 5]]).all()
    assert q[0, 3] == 127 and (q[1] == 127).all() and q[3, 7] == 127 and q[5, cols // 2] == 127


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


@pytest.mark.parametrize("T,H", [(128, 4096), (4096, 4096), (300, 5120), (9, 4100)])
def test_add_rmsnorm_quant_matches_the_two_step_composition(lib, T, H):
    """Fused kernel == cuda_add_rmsnorm followed by cuda_quantize_weights_per_row,
    both on the GPU (the composition it replaces), with a NaN and an inf row."""
    banner(f"add+rmsnorm+int8 vs composition T={T} H={H}")
    x = f16(RNG.standard_t(3, (T, H)) * 3)
    r = f16(RNG.standard_normal((T, H)) * 2)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    x[0, 5] = 0x7E00
    r[T - 1, H // 2] = 0x7C00
    q, s, ro = run_norm_quant(lib, x, w, 1e-5, residual=r)
    xb, rb, wb, yb, rob = dev(x), dev(r), dev(w), empty(x.nbytes), empty(x.nbytes)
    ok(lib.cuda_add_rmsnorm(yb.vp, rob.vp, xb.vp, rb.vp, wb.vp, T, H, C.c_float(1e-5)))
    q2b, s2b = empty(x.size), empty(4 * T)
    ok(lib.cuda_quantize_weights_per_row(q2b.vp, s2b.vp, yb.vp, T, H))
    assert_bits_equal(ro, get(rob, np.uint16, (T, H)), "residual_out")
    assert_bits_equal(q, get(q2b, np.int8, (T, H)), "codes")
    assert_bits_equal(s.view(np.uint32), get(s2b, np.uint32, (T,)), "scales")


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


@pytest.mark.parametrize("T,H", [(8, 4096), (6, 5120), (6, 4100), (2048, 4096)])
def test_norm_quant_rows_with_nan_and_inf(lib, ora, T, H):
    """RMSNorm + int8 (and the residual-add form) over rows holding a NaN or an
    inf: a NaN makes the whole normed row NaN (scale 1, codes +127); an inf makes
    r = 0, so the inf element normalises to NaN (+127) and the rest to 0."""
    banner(f"norm+int8 rows with NaN and inf T={T} H={H}")
    x = f16(RNG.standard_normal((T, H)))
    r = f16(RNG.standard_normal((T, H)) * 2)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    x[0, 1] = 0x7E00
    x[1, H - 1] = 0x7C00
    x[2, 0], x[2, 5] = 0xFC00, 0x7C00
    x[T - 1, H // 3] = 0x7C01
    r[3, 17] = 0xFE00                          # the residual's NaN reaches the sum
    q, s = run_norm_quant(lib, x, w, 1e-5)
    qw, sw = ora.rmsnorm_quant(x, w, 1e-5)
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")
    assert (q[0] == 127).all() and q[1, H - 1] == 127 and (q[1, :H - 1] == 0).all()
    q, s, ro = run_norm_quant(lib, x, w, 1e-5, residual=r)
    qw, sw, row = ora.add_rmsnorm_quant(x, r, w, 1e-5)
    # NaN payloads are not specified (the GPU keeps a quieted input payload,
    # the oracle writes 0x7E00): NaN positions must agree, other bits exactly.
    nan_g, nan_w = (ro & 0x7FFF) > 0x7C00, (row & 0x7FFF) > 0x7C00
    assert (nan_g == nan_w).all(), "residual_out NaN positions"
    assert_bits_equal(ro[~nan_w], row[~nan_w], "residual_out")
    assert_bits_equal(s.view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(q, qw, "codes")
    assert (q[3] == 127).all()


@pytest.mark.parametrize("n", [4096, 12345])
def test_per_tensor_quant_with_nan_and_inf(lib, ora, n):
    banner(f"per-tensor quant with NaN n={n}")
    x = f16(RNG.uniform(-1, 1, n) * 3)
    x[[5, n - 2]] = [0x7E00, 0xFC01]
    xb, qb, sb = dev(x), empty(n), empty(4)
    ok(lib.cuda_quantize_per_tensor(qb.vp, sb.vp, xb.vp, n), "quant tensor")
    qw, sw = ora.quant_tensor(x)
    assert np.isfinite(sw[0])
    assert_bits_equal(get(sb, np.float32, (1,)).view(np.uint32), sw.view(np.uint32), "scale")
    assert_bits_equal(get(qb, np.int8, (n,)), qw, "codes")
    x[7] = 0x7C00                              # and with an inf: scale inf
    xb2, qb2, sb2 = dev(x), empty(n), empty(4)
    ok(lib.cuda_quantize_per_tensor(qb2.vp, sb2.vp, xb2.vp, n), "quant tensor")
    qw, sw = ora.quant_tensor(x)
    assert np.isinf(sw[0])
    assert_bits_equal(get(sb2, np.float32, (1,)).view(np.uint32), sw.view(np.uint32), "scale")
    assert_bits_equal(get(qb2, np.int8, (n,)), qw, "codes")


@pytest.mark.parametrize("K,N", [(128, 64), (100, 33)])
def test_per_column_quant_with_nan_and_inf(lib, ora, K, N):
    banner(f"per-column quant with NaN {K}x{N}")
    x = np.ascontiguousarray(nonfinite_rows(N, K).T)   # the special cases down columns
    xb, qb, sb = dev(x), empty(x.size), empty(4 * N)
    ok(lib.cuda_quantize_weights(qb.vp, sb.vp, xb.vp, K, N), "quant cols")
    qw, sw = ora.quant_cols(x)
    assert_bits_equal(get(sb, np.float32, (N,)).view(np.uint32), sw.view(np.uint32), "scales")
    assert_bits_equal(get(qb, np.int8, (K, N)), qw, "codes")


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
