"""RMSNorm / add+RMSNorm on the GPU vs the oracle: bit-exact.

The row statistic is RN_f32 of the exact sum of squares on both sides and all
other steps are single IEEE operations, so fp16 and bf16 outputs must match
the oracle bit for bit, at every shape and for both the register-resident
and the element-wise kernels.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(7))

SHAPES = [(1, 4096), (7, 4096), (64, 4096), (300, 5120), (33, 2048), (5, 14336), (3, 13824),
          (2, 65536), (4, 4100), (4, 8), (17, 24), (2049, 4096), (600, 1000)]


def bits(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        from oracle.oracle import f32_to_bf16_bits

        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def run_rmsnorm(lib, x, w, eps, dtype, inplace=False, misalign=False):
    T, H = x.shape
    off = 2 if misalign else 0
    xb = empty(x.nbytes + off)
    xb.upload(np.concatenate([np.zeros(off // 2, np.uint16), x.ravel()]) if off else x)
    wb = dev(w)
    yb = xb if inplace else empty(x.nbytes + off)
    fn = lib.cuda_bf16_rmsnorm if dtype == "bf16" else lib.cuda_rmsnorm
    ok(fn(yb.offset(off), xb.offset(off), wb.vp, T, H, C.c_float(eps)), "rmsnorm")
    out = get(yb, np.uint16, (x.size + off // 2,))
    return out[off // 2:].reshape(T, H)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("T,H", SHAPES)
def test_rmsnorm_bit_exact(lib, ora, dtype, T, H):
    banner(f"rmsnorm {dtype} T={T} H={H}")
    x = bits(RNG.standard_normal((T, H)) * 3, dtype)
    w = bits(1 + 0.02 * RNG.standard_normal(H), dtype)
    got = run_rmsnorm(lib, x, w, 1e-5, dtype)
    assert_bits_equal(got, ora.rmsnorm(x, w, 1e-5, dtype), f"rmsnorm {dtype} {T}x{H}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rmsnorm_in_place_and_unaligned(lib, ora, dtype):
    banner(f"rmsnorm in-place/unaligned {dtype}")
    x = bits(RNG.standard_normal((9, 4096)), dtype)
    w = bits(1 + 0.02 * RNG.standard_normal(4096), dtype)
    want = ora.rmsnorm(x, w, 1e-6, dtype)
    assert_bits_equal(run_rmsnorm(lib, x, w, 1e-6, dtype, inplace=True), want, "in place")
    assert_bits_equal(run_rmsnorm(lib, x, w, 1e-6, dtype, misalign=True), want, "unaligned")


def adversarial_rows(H):
    """Rows whose exact sum of squares sits on (or next to) an fp32 rounding
    boundary, so the kernel's fp64 fast path cannot decide them."""
    rows = []
    for extra in ([], [2.0 ** -24], [2.0 ** -24, 2.0 ** -24]):
        r = np.zeros(H, np.float32)
        r[0], r[H // 2] = 2.0 ** 15, 8.0
        for j, v in enumerate(extra):
            r[H - 1 - j] = v
        rows.append(r)
    r = np.zeros(H, np.float32)
    r[3], r[H - 5] = 1.0, 2.0 ** -12
    rows.append(r)
    r = r.copy()
    r[7] = 2.0 ** -24
    rows.append(r)
    return np.stack(rows)


@pytest.mark.parametrize("T", [None, 2051])
@pytest.mark.parametrize("H", [4096, 5120, 4100])
def test_rmsnorm_exact_path_rows(lib, ora, H, T):
    """Rows that force the exact (integer-limb) reduction. Alone they run the
    kernel of small batches; scattered among T = 2051 ordinary rows they run the
    large-batch kernel, which loads the weights after the reduction and combines
    its partial sums with error-free steps before the exact fallback."""
    banner(f"rmsnorm exact-path rows H={H} T={T}")
    adv = bits(adversarial_rows(H), "f16")
    if T is None:
        x = adv
    else:
        x = bits(RNG.standard_normal((T, H)), "f16")
        at = np.sort(RNG.choice(T, adv.shape[0], replace=False))
        x[at] = adv
    w = bits(np.ones(H), "f16")
    got = run_rmsnorm(lib, x, w, 0.0, "f16")
    assert_bits_equal(got, ora.rmsnorm(x, w, 0.0), "adversarial")


def run_add_rmsnorm(lib, x, r, w, eps, dtype, inplace=False):
    T, H = x.shape
    xb, rb, wb = dev(x), dev(r), dev(w)
    yb = xb if inplace else empty(x.nbytes)
    rob = rb if inplace else empty(x.nbytes)
    fn = lib.ng_bf16_add_rmsnorm if dtype == "bf16" else lib.cuda_add_rmsnorm
    ok(fn(yb.vp, rob.vp, xb.vp, rb.vp, wb.vp, T, H, C.c_float(eps)), "add_rmsnorm")
    return get(yb, np.uint16, (T, H)), get(rob, np.uint16, (T, H))


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("T,H", [(1, 4096), (64, 4096), (257, 5120), (5, 4100), (2, 65536), (1030, 2048),
                                 (4096, 4096), (4099, 4096), (1537, 5120), (2048, 5120), (6200, 5120)])
@pytest.mark.parametrize("inplace", [False, True])
def test_add_rmsnorm_bit_exact(lib, ora, dtype, T, H, inplace):
    banner(f"add_rmsnorm {dtype} T={T} H={H} inplace={inplace}")
    x = bits(RNG.standard_normal((T, H)), dtype)
    r = bits(RNG.standard_normal((T, H)) * 2, dtype)
    w = bits(1 + 0.02 * RNG.standard_normal(H), dtype)
    y, ro = run_add_rmsnorm(lib, x, r, w, 1e-5, dtype, inplace)
    y_want, ro_want = ora.add_rmsnorm(x, r, w, 1e-5, dtype)
    assert_bits_equal(ro, ro_want, "residual_out")
    assert_bits_equal(y, y_want, "normed")


@pytest.mark.parametrize("T", [None, 4101])
def test_add_rmsnorm_exact_path_rows(lib, ora, T):
    """Rows that force the exact (integer-limb) reduction; T=4101 runs them
    through the several-rows-per-wave kernel of large prefill batches, with the
    adversarial rows scattered among ordinary ones and a partial last wave."""
    banner(f"add_rmsnorm exact-path rows T={T}")
    H = 4096
    adv = bits(adversarial_rows(H), "f16")
    if T is None:
        x = adv
    else:
        x = bits(RNG.standard_normal((T, H)), "f16")
        at = np.sort(RNG.choice(T, adv.shape[0], replace=False))
        x[at] = adv
    r = np.zeros_like(x)
    w = bits(np.ones(H), "f16")
    y, ro = run_add_rmsnorm(lib, x, r, w, 0.0, "f16")
    y_want, ro_want = ora.add_rmsnorm(x, r, w, 0.0)
    assert_bits_equal(ro, ro_want, "residual_out")
    assert_bits_equal(y, y_want, "normed")


def assert_bits_equal_nan(got, want, dtype, what):
    """Bit-exact except NaN payloads, which are not specified: NaN positions
    must agree."""
    inf = 0x7F80 if dtype == "bf16" else 0x7C00
    nan_g, nan_w = (got & 0x7FFF) > inf, (want & 0x7FFF) > inf
    assert (nan_g == nan_w).all(), f"{what}: NaN positions differ at {np.argwhere(nan_g != nan_w)[:5].tolist()}"
    assert_bits_equal(got[~nan_w], want[~nan_w], what)


def nonfinite_inputs(T, H, dtype):
    """Ordinary rows, plus rows holding an inf, a -inf, a NaN, and both. An inf
    makes the sum of squares inf, so r = 1 / sqrt(inf) = 0: finite values
    normalise to +-0 and the inf to NaN. A NaN makes the whole row NaN."""
    inf, ninf, nan = (0x7F80, 0xFF80, 0x7FC0) if dtype == "bf16" else (0x7C00, 0xFC00, 0x7E00)
    x = bits(RNG.standard_normal((T, H)), dtype)
    r = bits(RNG.standard_normal((T, H)) * 2, dtype)
    x[0, 1] = inf
    x[1, H - 1] = ninf
    x[2, H // 2] = nan
    x[3, 0], x[3, 9] = inf, nan
    x[T - 1, 7] = inf
    r[4, 3] = ninf                     # reaches the residual sum
    return x, r


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("T,H", [(6, 4096), (2050, 4096), (6, 5120), (6, 4100), (4096, 4096), (1600, 5120)])
def test_norm_rows_with_inf_and_nan(lib, ora, dtype, T, H):
    """RMSNorm and add+RMSNorm over rows holding infinities and NaNs, through
    every kernel shape (small and large batches, several waves per row, the
    element-wise kernel, several rows per wave)."""
    banner(f"rmsnorm / add_rmsnorm rows with inf and NaN {dtype} T={T} H={H}")
    x, r = nonfinite_inputs(T, H, dtype)
    w = bits(1 + 0.02 * RNG.standard_normal(H), dtype)
    got = run_rmsnorm(lib, x, w, 1e-5, dtype)
    want = ora.rmsnorm(x, w, 1e-5, dtype)
    assert_bits_equal_nan(got, want, dtype, "rmsnorm")
    y, ro = run_add_rmsnorm(lib, x, r, w, 1e-5, dtype)
    y_want, ro_want = ora.add_rmsnorm(x, r, w, 1e-5, dtype)
    assert_bits_equal_nan(ro, ro_want, dtype, "residual_out")
    assert_bits_equal_nan(y, y_want, dtype, "normed")
