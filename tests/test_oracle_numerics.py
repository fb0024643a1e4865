"""Pins the CPU oracle (oracle/ng_oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own code: exact rational arithmetic
(fractions), numpy's IEEE float32/float16 operations, fp64 closed forms,
invariants (scale invariance, identity rotation, norm preservation), and the
known-answer tests of the reference's Go suite (tests/kernels_test.go,
tests/quantize_test.go, tests/e2e/real_inference_test.go), restated.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

RNG = np.random.Generator(np.random.PCG64(1234))


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16v(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def ulp16(v):
    """binary16 ulp at |v| (subnormal spacing below 2^-14)."""
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -14)))
    return 2.0 ** (e - 10)


def rn_f32_exact(S: Fraction) -> np.float32:
    """Round a non-negative rational to float32, ties to even, exactly."""
    f0 = np.float32(float(S))
    best = None
    for c in (np.nextafter(f0, np.float32(-np.inf)), f0, np.nextafter(f0, np.float32(np.inf))):
        if not np.isfinite(c) or c < 0:
            continue
        d = abs(Fraction(float(c)) - S)
        key = (d, int(np.float32(c).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def exact_sumsq(vals) -> np.float32:
    return rn_f32_exact(sum((Fraction(float(v)) ** 2 for v in vals), Fraction(0)))


# --------------------------------------------------------------- formats

def test_f16_widening_exhaustive(ora):
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([ora.lib().ora_f16_to_f32(int(v)) for v in h], np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f16_rounding_matches_numpy_including_ties(ora):
    finite = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = (finite[:-1] + finite[1:]) / np.float32(2)  # exact midpoints: tie cases
    x = np.concatenate([mids, -mids, RNG.standard_normal(20000).astype(np.float32) * 1000,
                        np.float32([65504, 65519.99, 65520, 1e-8, 2.0 ** -25, 2.0 ** -24, 0.0, -0.0])])
    got = np.array([ora.lib().ora_f32_to_f16(float(v)) for v in x], np.uint16)
    assert (got == x.astype(np.float16).view(np.uint16)).all()


def test_bf16_rounding_matches_torch(ora):
    torch = pytest.importorskip("torch")
    x = np.concatenate([RNG.standard_normal(50000).astype(np.float32) * 10.0 ** RNG.integers(-20, 20, 50000),
                        np.float32([0.0, -0.0, 1.0, 3.4e38, 1e-40])]).astype(np.float32)
    b = x.view(np.uint32)
    ties = ((b & 0xFFFF0000) | 0x8000).view(np.float32)  # exact bf16 midpoints
    x = np.concatenate([x, ties])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([ora.lib().ora_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert (got == want).all()
    assert (ora.f32_to_bf16_bits(x) == want).all()


# --------------------------------------------------------------- sum of squares

@pytest.mark.parametrize("n", [1, 2, 7, 64, 257, 4096])
def test_sumsq_is_correctly_rounded_exact_sum_fp16_values(ora, n):
    for _ in range(3):
        v = f16v(f16(RNG.standard_normal(n) * 10.0 ** RNG.integers(-3, 3, n)))
        assert ora.sumsq(v) == exact_sumsq(v)


def test_sumsq_add_domain_values(ora):
    # s = RN_f32(a + b) of fp16 a, b: the add+RMSNorm statistic domain.
    a = f16v(f16(RNG.standard_normal(512)))
    b = f16v(f16(RNG.standard_normal(512) * 2))
    s = (a + b).astype(np.float32)
    assert ora.sumsq(s) == exact_sumsq(s)


@pytest.mark.parametrize(
    "vals, expect",
    [
        # exact sum 2^30 + 2^6 is an fp32 tie -> even (2^30)
        ([2.0 ** 15, 8.0], 2.0 ** 30),
        # 2^30 + 2^6 + 2^-48: above the tie, rounds up; fp64 alone loses the 2^-48
        ([2.0 ** 15, 8.0, 2.0 ** -24], 2.0 ** 30 + 2.0 ** 7),
        # 1 + 2^-24 is a tie -> 1; one more 2^-48 term breaks it upwards
        ([1.0, 2.0 ** -12], 1.0),
        ([1.0, 2.0 ** -12, 2.0 ** -24], 1.0 + 2.0 ** -23),
    ],
)
def test_sumsq_adversarial_ties(ora, vals, expect):
    v = np.float32(vals)
    assert float(ora.sumsq(v)) == expect
    assert exact_sumsq(v) == np.float32(expect)
    ora.set_exact_only(True)
    try:
        assert float(ora.sumsq(v)) == expect
    finally:
        ora.set_exact_only(False)


def test_sumsq_fast_path_agrees_with_exact_only(ora):
    rows = [f16v(f16(RNG.standard_normal(4096) * 10.0 ** RNG.integers(-4, 4, 4096))) for _ in range(20)]
    fast = [ora.sumsq(r) for r in rows]
    ora.set_exact_only(True)
    try:
        slow = [ora.sumsq(r) for r in rows]
    finally:
        ora.set_exact_only(False)
    assert fast == slow


def test_sumsq_off_grid_values_fall_back_to_fp64(ora):
    v = np.float32([1e-30, 3.0, 4.0])  # 1e-30 is not on the 2^-24 grid
    assert ora.sumsq(v) == np.float32(25.0)


# --------------------------------------------------------------- RMSNorm

def rmsnorm64(x, w, eps):
    x = np.asarray(x, np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(w, np.float64)


@pytest.mark.parametrize("H", [8, 100, 2048, 4096, 5120])
def test_rmsnorm_within_one_ulp_of_fp64(ora, H):
    x = f16(RNG.standard_normal((16, H)) * 3)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    y = f16v(ora.rmsnorm(x, w, 1e-5))
    ref = rmsnorm64(f16v(x), f16v(w), 1e-5)
    assert (np.abs(y - ref) <= ulp16(ref)).all()


def test_rmsnorm_reference_ramp_kat(ora):
    # tests/kernels_test.go:19-102: H=4096, x_i = 0.001 i, w = 1, eps = 1e-6
    # (Llama-7B preset), fp32 host values converted to fp16 by CopyToDevice.
    H = 4096
    xin = (np.arange(H, dtype=np.float32) * np.float32(0.001)).astype(np.float32)
    x = f16(xin)
    w = f16(np.ones(H))
    y = f16v(ora.rmsnorm(x, w, 1e-6))
    # The Go test's expectation uses the fp32 inputs (before fp16 rounding).
    ss = np.sum(xin.astype(np.float64) ** 2)
    r = 1.0 / np.sqrt(ss / H + 1e-6)
    exp = (xin.astype(np.float64) * r).astype(np.float32)
    nz = exp != 0
    rel = np.abs(y[nz] - exp[nz]) / np.abs(exp[nz])
    assert (rel > 0.002).sum() < 10
    # tighter: within one fp16 ulp of the fp64 value on the fp16 inputs
    ref = rmsnorm64(f16v(x), np.ones(H), 1e-6)
    assert (np.abs(y - ref) <= ulp16(ref)).all()


def test_rmsnorm_scale_invariance_bit_exact(ora):
    # eps = 0: scaling x by 2 scales sum x^2 by 4 exactly, r by 1/2 exactly.
    x = f16(RNG.standard_normal((8, 512)))
    w = f16(1 + 0.1 * RNG.standard_normal(512))
    assert (ora.rmsnorm(x, w, 0.0) == ora.rmsnorm(f16(f16v(x) * 2), w, 0.0)).all()


def test_rmsnorm_unit_weight_gives_unit_rms(ora):
    x = f16(RNG.standard_normal((4, 4096)) * 7)
    y = f16v(ora.rmsnorm(x, f16(np.ones(4096)), 0.0)).astype(np.float64)
    assert np.allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, atol=2e-3)


def test_rmsnorm_bf16_within_one_ulp(ora):
    H = 5120
    xb = ora.f32_to_bf16_bits(RNG.standard_normal((8, H)).astype(np.float32))
    wb = ora.f32_to_bf16_bits((1 + 0.02 * RNG.standard_normal(H)).astype(np.float32))
    y = ora.bf16_bits_to_f32(ora.rmsnorm(xb, wb, 1e-5, "bf16"))
    ref = rmsnorm64(ora.bf16_bits_to_f32(xb), ora.bf16_bits_to_f32(wb), 1e-5)
    ulp = 2.0 ** (np.floor(np.log2(np.abs(ref))) - 7)
    assert (np.abs(y - ref) <= ulp).all()


def test_add_rmsnorm_residual_exact_and_norm_close(ora):
    H = 4096
    x = f16(RNG.standard_normal((8, H)))
    res = f16(RNG.standard_normal((8, H)) * 2)
    y, ro = ora.add_rmsnorm(x, res, f16(1 + 0.02 * RNG.standard_normal(H)), 1e-5)
    s32 = f16v(x) + f16v(res)
    assert (ro == f16(s32)).all()
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    y, ro = ora.add_rmsnorm(x, res, w, 1e-5)
    s64 = f16v(x).astype(np.float64) + f16v(res)
    r = 1.0 / np.sqrt(np.mean(s64 * s64, axis=-1, keepdims=True) + 1e-5)
    ref = f16v(ro).astype(np.float64) * r * f16v(w)
    assert (np.abs(f16v(y) - ref) <= ulp16(ref)).all()


# --------------------------------------------------------------- element-wise

def test_silu_all_fp16_inputs_within_one_ulp(ora):
    h = np.arange(0, 65536, dtype=np.uint16)
    v = h.view(np.float16).astype(np.float64)
    h = h[np.isfinite(v)]
    v = v[np.isfinite(v)]
    y = f16v(ora.elementwise("silu", h)).astype(np.float64)
    with np.errstate(over="ignore"):
        ref = v / (1.0 + np.exp(-v))
    ok = np.abs(y - ref) <= ulp16(ref)
    assert ok.all(), np.flatnonzero(~ok)[:5]


def test_silu_reference_ramp_kat(ora):
    # tests/kernels_test.go:108-152: I = 11008, x_i = (i - 5504) * 0.01, first 100 within 1e-4.
    n = 11008
    xin = (np.arange(n, dtype=np.float32) - np.float32(n // 2)) * np.float32(0.01)
    y = f16v(ora.elementwise("silu", f16(xin)))
    x64 = xin[:100].astype(np.float64)
    assert (np.abs(y[:100] - x64 / (1 + np.exp(-x64))) < 1e-4).all()


def test_silu_mul_within_one_ulp(ora):
    g = f16(RNG.standard_normal(100000) * 4)
    u = f16(RNG.standard_normal(100000))
    y = f16v(ora.elementwise("silu_mul", g, u)).astype(np.float64)
    gv, uv = f16v(g).astype(np.float64), f16v(u).astype(np.float64)
    ref = gv / (1 + np.exp(-gv)) * uv
    assert (np.abs(y - ref) <= ulp16(ref)).all()


def test_add_mul_scale_exact(ora):
    a = f16(RNG.standard_normal(100000) * 100)
    b = f16(RNG.standard_normal(100000))
    assert (ora.elementwise("add", a, b) == f16(f16v(a) + f16v(b))).all()
    assert (ora.elementwise("mul", a, b) == f16(f16v(a) * f16v(b))).all()
    assert (ora.elementwise("scale", a, s=0.37) == f16(f16v(a) * np.float32(0.37))).all()


def test_add_reference_ramp_kat(ora):
    # tests/kernels_test.go:215-274: a_i = 0.001 i, b_i = 0.001 (4096 - i), abs 0.01.
    n = 4096
    a = np.arange(n, dtype=np.float32) * np.float32(0.001)
    b = (np.float32(n) - np.arange(n, dtype=np.float32)) * np.float32(0.001)
    c = f16v(ora.elementwise("add", f16(a), f16(b)))
    assert (np.abs(c - (a + b)) > 0.01).sum() < 10


def test_bf16_elementwise(ora):
    a = ora.f32_to_bf16_bits(RNG.standard_normal(50000).astype(np.float32) * 3)
    b = ora.f32_to_bf16_bits(RNG.standard_normal(50000).astype(np.float32))
    av, bv = ora.bf16_bits_to_f32(a), ora.bf16_bits_to_f32(b)
    assert (ora.elementwise("add", a, b, dtype="bf16") == ora.f32_to_bf16_bits(av + bv)).all()
    assert (ora.elementwise("mul", a, b, dtype="bf16") == ora.f32_to_bf16_bits(av * bv)).all()
    y = ora.bf16_bits_to_f32(ora.elementwise("silu_mul", a, b, dtype="bf16")).astype(np.float64)
    ref = av / (1 + np.exp(-av.astype(np.float64))) * bv
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref), 1e-38))) - 7)
    assert (np.abs(y - ref) <= ulp).all()


# --------------------------------------------------------------- RoPE

def rope64(x, pos, inv32, style):
    """fp64 rotation at the fp32 angle fl(pos * inv) that defines the kernel."""
    x = np.asarray(x, np.float64)
    D = x.shape[-1]
    half = D // 2
    ang = (pos.astype(np.float32)[:, None] * inv32[None, :]).astype(np.float64)  # fp32 product
    c = np.cos(ang)[:, None, :]
    s = np.sin(ang)[:, None, :]
    if style == 1:
        x1, x2 = x[..., 0::2], x[..., 1::2]
    else:
        x1, x2 = x[..., :half], x[..., half:]
    y1 = x1 * c - x2 * s
    y2 = x1 * s + x2 * c
    y = np.empty_like(x)
    if style == 1:
        y[..., 0::2], y[..., 1::2] = y1, y2
    else:
        y[..., :half], y[..., half:] = y1, y2
    return y


def test_rope_inv_freq_matches_closed_form(ora):
    for D, theta in [(64, 1e4), (128, 1e6), (128, 1e4), (256, 5e5)]:
        inv = ora.rope_inv_freq(D, theta)
        ref = theta ** (-(2.0 * np.arange(D // 2)) / D)
        assert np.allclose(inv, ref, rtol=3e-7, atol=0)


@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("D,theta,maxpos", [(128, 1e6, 4096), (64, 1e4, 128), (128, 1e6, 32768)])
def test_rope_within_one_ulp_of_fp64(ora, style, D, theta, maxpos):
    T, nh = 32, 4
    x = f16(RNG.standard_normal((T, nh, D)))
    pos = RNG.integers(0, maxpos, T).astype(np.int32)
    y = f16v(ora.rope(x, pos, style, theta))
    ref = rope64(f16v(x), pos, ora.rope_inv_freq(D, theta), style)
    assert (np.abs(y - ref) <= ulp16(ref)).all()


def test_rope_position_zero_is_identity(ora):
    x = f16(RNG.standard_normal((4, 8, 128)))
    for style in (0, 1):
        assert (ora.rope(x, np.zeros(4, np.int32), style, 1e4) == x).all()


def test_rope_preserves_pair_norms(ora):
    x = f16(RNG.standard_normal((16, 8, 128)))
    pos = RNG.integers(0, 4096, 16).astype(np.int32)
    y = f16v(ora.rope(x, pos, 0, 1e4)).astype(np.float64)
    xv = f16v(x).astype(np.float64)
    n_in = xv[..., :64] ** 2 + xv[..., 64:] ** 2
    n_out = y[..., :64] ** 2 + y[..., 64:] ** 2
    assert np.allclose(n_out, n_in, rtol=4e-3, atol=1e-3)


def test_rope_matches_reference_golden_formula(ora):
    # scripts/generate_golden.py:55-77 (compute_rope): split-half, theta 1e4,
    # positions 0..S-1, evaluated here in fp64.
    S, nh, D = 64, 4, 128
    x = f16(RNG.standard_normal((S, nh, D)))
    xv = f16v(x).astype(np.float64)
    inv = 1.0 / (10000 ** (np.arange(0, D, 2) / D))
    fr = np.arange(S)[:, None] * inv[None, :]
    c, s = np.cos(fr)[:, None, :], np.sin(fr)[:, None, :]
    x1, x2 = xv[..., :D // 2], xv[..., D // 2:]
    ref = np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)
    y = f16v(ora.rope(x, np.arange(S, dtype=np.int32), 0, 1e4))
    assert ((np.abs(y - ref) <= 1e-2) | (np.abs(y - ref) <= 2 * ulp16(ref))).all()


# --------------------------------------------------------------- quantisation

def ieee_codes(v, scale):
    z = np.float32(v) / np.float32(scale)  # numpy float32 division is IEEE
    return np.clip(np.rint(z), -127, 127).astype(np.int8)


def test_quant_all_fp16_values_per_row(ora):
    h = np.arange(0, 0x7C00, dtype=np.uint16)          # every finite non-negative pattern
    allv = np.concatenate([h, h | 0x8000])               # and its negation
    rows = allv[: (allv.size // 496) * 496].reshape(-1, 496)
    q, s = ora.quant_rows(rows)
    v = f16v(rows)
    m = np.abs(v).max(axis=1)
    exp_s = (m / np.float32(127)).astype(np.float32)
    exp_s[exp_s == 0] = 1
    assert (s.view(np.uint32) == exp_s.view(np.uint32)).all()
    assert (q == ieee_codes(v, exp_s[:, None])).all()


@pytest.mark.parametrize("scale", [1.0, 0.01, 2.0 ** -20, 1 / 127, 3.1e-3])
def test_quant_exhaustive_fp16_at_fixed_scales(ora, scale):
    # A row holding every finite fp16 value whose magnitude is at most 127 * scale
    # plus one element at exactly 127 * scale (rounded to fp16) fixes the scale.
    h = np.arange(0, 0x7C00, dtype=np.uint16)
    v = f16v(h)
    m = np.float32(np.float16(127 * scale))
    keep = v <= m
    row = np.concatenate([h[keep], h[keep] | 0x8000])
    q, s = ora.quant_rows(row[None, :])
    sc = np.float32(m) / np.float32(127)
    assert s[0] == sc
    assert (q[0] == ieee_codes(f16v(row), sc)).all()


def test_quant_invariants(ora):
    x = f16(RNG.standard_t(3, (64, 1024)) * 5)
    q, s = ora.quant_rows(x)
    v = f16v(x)
    assert (np.abs(q.astype(int)) <= 127).all()
    am = np.abs(v).argmax(axis=1)
    assert (np.abs(q[np.arange(64), am]) == 127).all()
    qn, sn = ora.quant_rows(f16(-v))
    assert (qn == -q).all() and (sn == s).all()
    z, sz = ora.quant_rows(np.zeros((2, 64), np.uint16))
    assert (z == 0).all() and (sz == 1).all()
    # reconstruction error at most half a step
    assert (np.abs(q * s[:, None].astype(np.float64) - v) <= s[:, None] / 2 * (1 + 1e-6)).all()


def ref_nonfinite_codes(v, axis):
    """The reference's rule restated with numpy's NaN-skipping routines: the
    absmax is an fmaxf reduction from 0 (block_reduce_max, quantize.cu:24-50:
    NaNs skipped, like np.fmax), scale = m / 127 (1 when 0), and the codes are
    fmaxf(-127, fminf(127, rint(v / scale))) (quantize.cu:313): np.fmin / np.fmax
    return the non-NaN operand exactly as C's fminf / fmaxf do."""
    a = np.abs(v)
    m = np.fmax.reduce(np.where(np.isnan(a), np.float32(0), a), axis=axis, keepdims=True).astype(np.float32)
    s = (m / np.float32(127)).astype(np.float32)
    s[s == 0] = 1
    with np.errstate(invalid="ignore", divide="ignore"):
        z = np.rint((v / s).astype(np.float32))
    q = np.fmax(np.float32(-127), np.fmin(np.float32(127), z)).astype(np.int8)
    return q, np.squeeze(s, axis=axis)


def nonfinite_rows(rng, rows, cols):
    x = f16(rng.standard_normal((rows, cols)) * rng.uniform(0.1, 10, (rows, 1)))
    x[0, 3] = 0x7E00                     # one quiet NaN
    x[1, :] = 0x7E00                     # all NaN: scale 1, every code +127
    x[2, 5], x[2, 9] = 0x7C01, 0xFE00    # signalling and negative NaNs
    x[3, 7] = 0x7C00                     # +inf: scale inf
    x[4, 0], x[4, 1] = 0xFC00, 0x7E00    # -inf and a NaN
    return x


def test_quant_nan_and_inf_rows_follow_the_reference_rule(ora):
    x = nonfinite_rows(RNG, 8, 96)
    v = f16v(x)
    q, s = ora.quant_rows(x)
    qw, sw = ref_nonfinite_codes(v, 1)
    assert (s.view(np.uint32) == sw.view(np.uint32)).all()
    assert (q == qw).all()
    # the cases spelled out: NaN elements +127, finite codes untouched by them
    assert q[0, 3] == 127 and np.isfinite(s[0]) and s[0] == np.float32(np.abs(np.delete(v[0], 3)).max()) / 127
    assert (q[1] == 127).all() and s[1] == 1
    assert q[2, 5] == 127 and q[2, 9] == 127
    assert np.isinf(s[3]) and q[3, 7] == 127 and (np.delete(q[3], 7) == 0).all()
    assert np.isinf(s[4]) and q[4, 0] == 127 and q[4, 1] == 127
    # per tensor and per column take the same rule
    qt, st = ora.quant_tensor(x[0])
    qtw, stw = ref_nonfinite_codes(v[0], 0)
    assert st[0] == stw and (qt == qtw).all()
    qc, sc = ora.quant_cols(np.ascontiguousarray(x.T))
    qcw, scw = ref_nonfinite_codes(np.ascontiguousarray(v.T), 0)
    assert (sc.view(np.uint32) == scw.view(np.uint32)).all() and (qc == qcw).all()


def test_norm_quant_with_nan_and_inf_inputs(ora):
    """A NaN in x makes every normed value NaN (scale 1, codes +127); an inf makes
    ss = inf, r = 0, so finite values normalise to 0 and the inf to NaN (+127)."""
    x = f16(RNG.standard_normal((3, 64)))
    w = f16(1 + 0.02 * RNG.standard_normal(64))
    x[0, 10] = 0x7E00
    x[1, 20] = 0x7C00
    q, s = ora.rmsnorm_quant(x, w, 1e-5)
    assert s[0] == 1 and (q[0] == 127).all()
    assert s[1] == 1 and q[1, 20] == 127 and (np.delete(q[1], 20) == 0).all()
    y = ora.rmsnorm(x, w, 1e-5)
    qw, sw = ref_nonfinite_codes(f16v(y), 1)
    assert (q == qw).all() and (s == sw).all()


@pytest.mark.parametrize("T,H", [(16, 96), (5, 4100), (3, 4096)])
def test_fused_norm_quant_equals_its_composition(ora, T, H):
    """The fused oracle functions equal the compositions they stand for, each
    part pinned on its own above: rmsnorm_quant == quant_rows(rmsnorm) and
    add_rmsnorm_quant == quant_rows(add_rmsnorm) with the same residual output,
    bit for bit, including rows with NaN and inf in x or in the residual, a
    zero row and a row whose sum overflows fp16."""
    x = f16(RNG.standard_normal((T, H)) * 3)
    r = f16(RNG.standard_normal((T, H)) * 2)
    w = f16(1 + 0.02 * RNG.standard_normal(H))
    x[0, 1] = 0x7E00                   # NaN in x
    x[1, H - 1] = 0x7C00               # +inf in x
    r[2, 3] = 0xFE00                   # NaN in the residual only
    x[T - 1, :] = 0                    # zero row (plain form) ...
    r[T - 1, :] = 0                    # ... and zero sum (residual form)
    if T > 4:
        x[3, 7], r[3, 7] = 0x7BFF, 0x7BFF  # 65504 + 65504 overflows to inf in the residual output
    q, sc = ora.rmsnorm_quant(x, w, 1e-5)
    qw, sw = ora.quant_rows(ora.rmsnorm(x, w, 1e-5))
    assert (sc.view(np.uint32) == sw.view(np.uint32)).all()
    assert (q == qw).all()
    q, sc, ro = ora.add_rmsnorm_quant(x, r, w, 1e-5)
    y, row = ora.add_rmsnorm(x, r, w, 1e-5)
    qw, sw = ora.quant_rows(y)
    assert (ro == row).all()
    assert (sc.view(np.uint32) == sw.view(np.uint32)).all()
    assert (q == qw).all()
    assert sc[T - 1] == 1 and (q[T - 1] == 0).all()


def test_quant_per_tensor_reference_kat(ora):
    # tests/quantize_test.go:20-87: U(-1, 1), n = 4096, scale within 0.01 of max/127,
    # round-trip error below 0.01.
    data = RNG.uniform(-1, 1, 4096).astype(np.float32)
    q, s = ora.quant_tensor(f16(data))
    assert abs(s[0] - np.abs(data).max() / 127) < 0.01
    assert np.abs(q * s[0] - data).max() < 0.01


def test_quant_per_column_reference_kat(ora):
    # tests/quantize_test.go:156-221: [128, 64] weights, per-column, recon error < 0.01.
    w = RNG.uniform(-1, 1, (128, 64)).astype(np.float32)
    q, s = ora.quant_cols(f16(w))
    assert np.abs(q * s[None, :] - f16v(f16(w))).max() < 0.01
    exp_s = (np.abs(f16v(f16(w))).max(axis=0) / np.float32(127)).astype(np.float32)
    assert (s == exp_s).all()
    assert (q == ieee_codes(f16v(f16(w)), exp_s[None, :])).all()


def test_dequant_exhaustive_codes(ora):
    codes = np.arange(-128, 128, dtype=np.int8)
    scales = np.float32([0.01, 1e-3, 7.3e-3, 2.0 ** -10, 0.5, 1.0])
    q = np.tile(codes, (scales.size, 1))
    out = ora.dequant(q, scales, "row")
    want = (q.astype(np.float32) * scales[:, None]).astype(np.float16).view(np.uint16)
    assert (out == want).all()
    outc = ora.dequant(q.T.copy(), scales, "col")
    assert (outc == want.T).all()
    outt = ora.dequant(codes, np.float32([0.01]), "tensor")
    assert (outt == (codes.astype(np.float32) * np.float32(0.01)).astype(np.float16).view(np.uint16)).all()


def test_dequant_reference_kat(ora):
    # tests/quantize_test.go:89-154: codes U{-128..127}, scale 0.01, abs 1e-3.
    codes = RNG.integers(-128, 128, 4096).astype(np.int8)
    out = f16v(ora.dequant(codes, np.float32([0.01]), "tensor"))
    assert (np.abs(out - codes * np.float32(0.01)) > 1e-3).sum() < 10


# --------------------------------------------------------------- loader bf16 -> fp16

def test_bf16_to_f16_trunc_every_pattern(ora):
    """loader.go:23-85 for all 65 536 bf16 inputs against an independent rule:
    round toward zero to fp16 (numpy's nearest conversion, stepped one ulp
    toward zero where it rounded away), except |x| >= 2^16 -> inf and
    NaN -> 0x7E00 with the sign."""
    h = np.arange(65536, dtype=np.uint16)
    got = ora.bf16_to_f16_trunc(h)
    x = ora.bf16_bits_to_f32(h)
    with np.errstate(over="ignore"):
        near = x.astype(np.float16)
    nb = near.view(np.uint16).astype(np.int32)
    away = np.abs(near.astype(np.float64)) > np.abs(x.astype(np.float64))
    want = np.where(away, nb - 1, nb)
    sign = (h & 0x8000).astype(np.int32)
    want = np.where(np.abs(x) >= 65536.0, sign | 0x7C00, want)
    want = np.where(np.isnan(x), sign | 0x7E00, want)
    assert (got == want.astype(np.uint16)).all()


def test_bf16_to_f16_trunc_reference_kat(ora):
    """TestBF16ToFP16Conversion (tests/model/loader_test.go:443-470): 1.0 -> 0x3C00, 0.0 -> 0."""
    assert ora.bf16_to_f16_trunc(np.array([0x3F80], np.uint16))[0] == 0x3C00
    assert ora.bf16_to_f16_trunc(np.array([0x0000], np.uint16))[0] == 0x0000


# --------------------------------------------------------------- int8-weight GEMM

def _gemm_int8_loops(a_bits, q, scale, transpose_b):
    """matmul.cu:169-244 written out element by element: w = fp16(float(q) *
    scale) in the stored layout, then C[m, n] = sum_k A[m, k] * w(k, n)."""
    a = a_bits.view(np.float16)
    M, K = a.shape
    N = q.shape[0] if transpose_b else q.shape[1]
    C = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = Fraction(0)
            for k in range(K):
                code = int(q[n, k] if transpose_b else q[k, n])
                w = np.float16(np.float32(code) * np.float32(scale[n]))
                acc += Fraction(float(a[m, k])) * Fraction(float(w))
            C[m, n] = float(acc)
    return C


@pytest.mark.parametrize("transpose_b", [False, True])
def test_gemm_int8_oracle_matches_loops(ora, transpose_b):
    M, K, N = 3, 7, 5
    a = RNG.standard_normal((M, K)).astype(np.float16).view(np.uint16)
    q = RNG.integers(-128, 128, (N, K) if transpose_b else (K, N)).astype(np.int8)
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    got = ora.gemm_int8(a, q, scale, transpose_b)
    want = _gemm_int8_loops(a, q, scale, transpose_b)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-15)


def test_gemm_int8_oracle_identity_rows_are_the_fp16_weights(ora):
    """A = I picks out the dequantized weights: C[m, n] = fp16(q[n, m] * s[n])
    (transpose_b), which is exact, so the scale index per row of B is pinned."""
    K = N = 16
    a = np.eye(K, dtype=np.float16).view(np.uint16)
    q = RNG.integers(-128, 128, (N, K)).astype(np.int8)
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    C = ora.gemm_int8(a, q, scale, True)
    w = (q.astype(np.float32) * scale[:, None]).astype(np.float16).astype(np.float64)
    assert (C == w.T).all()
    Ccol = ora.gemm_int8(a, q.T.copy(), scale, False)
    assert (Ccol == w.T).all()


def test_gemm_int8_oracle_reference_kat(ora):
    """TestGEMMINT8 (tests/matmul_test.go:98-179): [32,128] x [128,64], A U(-1,1),
    codes U{-128..127}, scales 0.01: the oracle (fp16 A and w) stays within the
    test's 5e-2 of the fp32 CPU matmul of the unrounded data."""
    M, K, N = 32, 128, 64
    A = RNG.random((M, K), dtype=np.float32) * 2 - 1
    q = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    scale = np.full(N, 0.01, np.float32)
    C = ora.gemm_int8(A.astype(np.float16).view(np.uint16), q, scale, False)
    ref = A @ (q.astype(np.float32) * scale[None, :])
    assert np.abs(C - ref).max() < 5e-2


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
def test_gemm_fp16_oracle_transposes(ora, ta, tb):
    M, K, N = 4, 6, 3
    a = RNG.standard_normal((K, M) if ta else (M, K)).astype(np.float16)
    b = RNG.standard_normal((N, K) if tb else (K, N)).astype(np.float16)
    got = ora.gemm_fp16(a.view(np.uint16), b.view(np.uint16), ta, tb)
    for m in range(M):
        for n in range(N):
            s = sum(Fraction(float(a[k, m] if ta else a[m, k])) * Fraction(float(b[n, k] if tb else b[k, n]))
                    for k in range(K))
            assert got[m, n] == pytest.approx(float(s), rel=1e-12, abs=1e-15)


# --------------------------------------------------------------- gather, softmax

def test_gather_reference_byte_pattern_kat(ora):
    # tests/e2e/real_inference_test.go:218-253: V=100, H=128 fp16, bytes i % 256, token 42.
    V, H = 100, 128
    table = (np.arange(V * H * 2) % 256).astype(np.uint8).view(np.uint16).reshape(V, H)
    row = ora.gather(table, np.int32([42]))
    b = row.view(np.uint8).ravel()
    off = 42 * H * 2
    assert all(b[i] == (off + i) % 256 for i in range(10))


def test_gather_bit_exact(ora):
    table = RNG.integers(0, 65536, (1000, 96)).astype(np.uint16)
    ids = RNG.integers(0, 1000, 300).astype(np.int32)
    assert (ora.gather(table, ids) == table[ids]).all()


def test_softmax_close_to_fp64(ora):
    x = f16(RNG.standard_normal((8, 1000)) * 4)
    y = f16v(ora.softmax(x)).astype(np.float64)
    xv = f16v(x).astype(np.float64)
    e = np.exp(xv - xv.max(axis=1, keepdims=True))
    ref = e / e.sum(axis=1, keepdims=True)
    assert (np.abs(y - ref) <= ulp16(ref)).all()


# --------------------------------------------------------------- fp32 golden path (TinyLlama config)

def test_tinyllama_fp32_golden_path(ora):
    """Config 1: the reference CPU golden formulas in fp32 (torch), fp32 oracle
    within 1e-5 relative (scripts/generate_golden.py:43-77)."""
    torch = pytest.importorskip("torch")
    from neurogrid_amd import workloads as W

    for key in ("tinyllama_t1", "tinyllama_t128"):
        cfg = W.CONFIGS[key]
        d = W.make_layer_inputs(cfg, seed=0, with_table=False)
        x, w = d["x"], d["w_attn"]
        y = ora.rmsnorm_f32(x, w, cfg.eps)
        xt, wt = torch.from_numpy(x), torch.from_numpy(w)
        var = xt.pow(2).mean(-1, keepdim=True)
        yt = (xt * torch.rsqrt(var + cfg.eps) * wt).numpy()
        assert np.allclose(y, yt, rtol=1e-5, atol=1e-6)
        g, u = d["gate"], d["up"]
        sm = ora.elementwise_f32("silu_mul", g, u)
        gt = torch.from_numpy(g)
        smt = (gt * torch.sigmoid(gt) * torch.from_numpy(u)).numpy()
        assert np.allclose(sm, smt, rtol=1e-5, atol=1e-6)
        for name, nh in (("q", cfg.nq), ("k", cfg.nkv)):
            xr = d[name]
            yr = ora.rope_f32(xr, d["pos"], 0, cfg.theta)
            ref = rope64(xr, d["pos"], ora.rope_inv_freq(cfg.D, cfg.theta), 0)
            assert np.allclose(yr, ref, rtol=1e-5, atol=1e-6)
