"""The benchmark's byte accounting and its one-GPU rule, on the CPU.

`value` and every roofline figure divide algorithmic bytes by a time, so the
per-kernel byte counts of neurogrid_amd/workloads.py are checked against the
figures of the measurement plan, which were worked out from the model shapes
independently of this code: per-layer totals of 738.2 MB (Mistral-7B
prefill), 11.6 MB (decode, T = 64), 1770.1 MB (Llama-2-13B prefill) and
406.9 MB (Mistral-Nemo bf16), and the Mistral-7B prefill column per kernel.
"""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

from neurogrid_amd import workloads as W

ROOT = Path(__file__).resolve().parent.parent

# MB (1e6 bytes) to 0.1, as the plan states them (rounded or truncated: within 0.1).
LAYER_MB = {"mistral7b_prefill": 738.2, "mistral7b_decode": 11.6, "llama2_13b_prefill": 1770.1,
            "mistral_nemo_bf16": 406.9}
M7P_KERNEL_MB = {"rmsnorm": 67.1, "add_rmsnorm": 134.2, "silu_mul": 352.3, "rope_q": 67.1, "rope_k": 16.8,
                 "add": 100.7, "gather": 67.1}
GATHER_MB = {"mistral7b_prefill": 67.1, "mistral_nemo_bf16": 41.9}


def near(nbytes: int, mb: float) -> bool:
    return 0 <= nbytes / 1e6 - mb < 0.1 or abs(nbytes / 1e6 - mb) <= 0.05


@pytest.mark.parametrize("key", sorted(LAYER_MB))
def test_layer_bytes_match_the_plan(key):
    b = W.layer_bytes(W.CONFIGS[key])
    assert near(sum(b[k] for k in W.LAYER_KERNELS), LAYER_MB[key])
    if key in GATHER_MB:
        assert near(b["gather"], GATHER_MB[key])


def test_mistral7b_prefill_kernel_bytes():
    b = W.layer_bytes(W.CONFIGS["mistral7b_prefill"])
    assert b.keys() == M7P_KERNEL_MB.keys()
    assert all(near(b[k], mb) for k, mb in M7P_KERNEL_MB.items()), b
    # SwiGLU, the roofline's kernel: three fp16 streams of 4096 x 14336.
    assert b["silu_mul"] == 352_321_536


def test_quant_bytes_match_the_plan():
    q = W.quant_bytes()
    assert near(q["rmsnorm_quant"], 50.4)
    assert near(q["dequant"], 176.2)


def test_bench_refuses_more_than_one_gpu():
    """More than one GPU is refused before the library is loaded."""
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)
    assert proc.returncode == 2
    line = json.loads(proc.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_bench_lists_its_modes():
    """Every mode of bench.py parses (--help exits before any GPU call)."""
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--help"], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)
    assert proc.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup", "--profile-pass", "--profile-decode", "--decode-only",
                 "--gemm-only", "--floors-only"):
        assert flag in proc.stdout, flag


def test_floor_kernels_compile_for_gfx950():
    """The access-pattern floor kernels bench.py times compile with hipRTC for
    gfx950 (compilation needs no GPU), so a GPU run never finds them broken."""
    import ctypes as C

    sys.path.insert(0, str(ROOT))
    import bench

    rtc = C.CDLL("libhiprtc.so")
    prog = C.c_void_p()
    assert rtc.hiprtcCreateProgram(C.byref(prog), bench.FLOOR_SRC.encode(), b"floors.hip", 0, None, None) == 0
    opts = (C.c_char_p * 2)(b"--offload-arch=gfx950", b"-O3")
    rc = rtc.hiprtcCompileProgram(prog, 2, opts)
    n = C.c_size_t()
    rtc.hiprtcGetCodeSize(prog, C.byref(n))
    rtc.hiprtcDestroyProgram(C.byref(prog))
    assert rc == 0 and n.value > 0
