"""The oracle against the reference's own CPU golden vectors.

Fixtures in tests/golden/reference_kernels/ were written by the reference's
scripts/generate_golden.py in --kernels-only --device cpu mode (torch fp16 on
the CPU, torch.manual_seed(42)); see tests/golden/gen_reference_golden.py.
The reference computes in fp16 dtype (rounding after each torch op); the
oracle rounds once, so agreement is to the stated tolerance: |d| <= 1e-2 or
|d| <= 2 ulp, with the exact-match rate reported.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

GOLD = Path(__file__).resolve().parent / "golden" / "reference_kernels"


def load(name):
    return np.fromfile(GOLD / name, dtype="<f4")


def f16(x):
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def ulp16(v):
    v = np.abs(np.asarray(v, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0 ** -14))) - 10)


def test_fixtures_are_fp16_values():
    for name in ["rmsnorm_input.bin", "rmsnorm_weight.bin", "silu_input.bin"]:
        v = load(name)
        assert (v.astype(np.float16).astype(np.float32) == v).all()


def test_rmsnorm_matches_reference_golden(ora):
    x, w, y = load("rmsnorm_input.bin"), load("rmsnorm_weight.bin"), load("rmsnorm_output.bin")
    assert x.size == 4096 and (w == 1).all()
    got = ora.f16_bits_to_f32(ora.rmsnorm(f16(x)[None, :], f16(w), 1e-6)).ravel()
    d = np.abs(got - y)
    assert ((d <= 1e-2) | (d <= 2 * ulp16(y))).all()
    assert (d <= ulp16(y)).all()          # in fact within one ulp
    assert (got == y).mean() > 0.95       # and mostly identical


def test_silu_matches_reference_golden(ora):
    x, y = load("silu_input.bin"), load("silu_output.bin")
    assert x.size == 11008
    got = ora.f16_bits_to_f32(ora.elementwise("silu", f16(x)))
    d = np.abs(got - y)
    assert ((d <= 1e-2) | (d <= 2 * ulp16(y))).all()
    assert (d <= ulp16(y)).all()
    # the reference's own golden tolerances (tests/golden_test.go:24-201)
    assert d.max() < 5e-3 and d.mean() < 1e-4 and (d > 1e-3).mean() < 0.01
