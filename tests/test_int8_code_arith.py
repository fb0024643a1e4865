"""The division-free int8 code of the GPU kernels, checked exhaustively on the
CPU: tests/int8_code_check.c replays its fp32 steps (qcode8 / qcode_int in
neurogrid_amd/csrc/ng_common.hpp) for every positive finite fp16 row absmax m
and every fp16 value v with |v| <= m, about 10^9 pairs, against the
reference's rule clamp(rint(v / s), -127, 127) with the IEEE quotient
(gpu/cuda/quantize.cu:292-313). A plain product v * (1/s) must be seen to fail
somewhere, so the check can tell the correction step from no correction."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_division_free_codes_exhaustive(tmp_path):
    exe = tmp_path / "int8_code_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-o", str(exe), str(HERE / "int8_code_check.c"),
                    "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    m = re.search(r"pairs (\d+) markstein_wrong (\d+) plain_wrong (\d+)", r.stdout)
    assert m, r.stdout + r.stderr
    pairs, wrong, plain = (int(g) for g in m.groups())
    assert pairs > 10 ** 9 and wrong == 0 and plain > 0, r.stdout
    assert r.returncode == 0, r.stdout
