"""The C++ host mirror of the reference's Go bindings
(neurogrid_amd/host/neurogrid_gpu.cpp, restating gpu/bindings/gpu.go) and the
reference's Go kernel tests restated over it (tests/host/host_test.cpp).

The CPU tests check that both are built, that the library exports every
wrapper the header declares and that the test program lists the restated Go
tests. The GPU test runs the program once, in its own process, and requires
every test in it to pass.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "neurogrid_amd" / "lib"
HOST_LIB = LIB / "libneurogrid_host.so"
HOST_TEST = LIB / "host_test"
HEADER = ROOT / "neurogrid_amd" / "host" / "neurogrid_gpu.hpp"

# The Go tests restated (tests/kernels_test.go, quantize_test.go,
# matmul_test.go, cgo_test.go, golden_test.go, e2e/real_inference_test.go) plus checks of
# the copy rounding, the bf16 wrappers and concurrent GEMMINT8 calls.
EXPECTED = [
    "TestDeviceInfo", "TestRMSNorm", "TestSiLU", "TestRMSNormGolden", "TestSiLUGolden", "TestRoPE", "TestAddKernel",
    "TestQuantizePerTensor", "TestDequantizePerTensor", "TestQuantizeWeights",
    "TestCopyFP16RoundToNearestEven", "TestEmbeddingLookup", "TestBF16Conversion",
    "TestCGOErrorHandling",
    "TestGEMMFP16", "TestGEMMTranspose", "TestGEMMINT8", "TestCGOOverheadValidation",
    "TestCGOConcurrentCalls", "TestConcurrentGEMMINT8", "TestCGOInitShutdown",
]


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    body = text[text.index("namespace neurogrid {"):]
    names = re.findall(r"^(?:Error|bool|void|Tensor|size_t)\s+(\w+)\(", body, re.M)
    return sorted(set(names))


def test_host_build_exports_every_wrapper():
    assert HOST_LIB.exists(), f"{HOST_LIB} not built (run __graft_entry__.build())"
    out = subprocess.run(["nm", "-DC", "--defined-only", str(HOST_LIB)], capture_output=True, text=True,
                         check=True).stdout
    defined = set(re.findall(r"neurogrid::(\w+)\(", out))
    declared = _declared_functions()
    assert len(declared) >= 27, declared
    missing = [n for n in declared if n not in defined]
    assert not missing, f"declared in neurogrid_gpu.hpp but not exported: {missing}"


def test_host_test_lists_the_restated_go_tests():
    assert HOST_TEST.exists(), f"{HOST_TEST} not built (run __graft_entry__.build())"
    out = subprocess.run([str(HOST_TEST), "--list"], capture_output=True, text=True, check=True, timeout=60).stdout
    assert out.split() == EXPECTED


def test_host_test_rejects_unknown_names():
    proc = subprocess.run([str(HOST_TEST), "TestNoSuchThing"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 2 and "unknown test TestNoSuchThing" in proc.stderr


@pytest.mark.gpu
def test_host_cpp_go_suite(lib):
    """All of host_test on device 0, in one child process."""
    print("host_test: the Go kernel and cgo tests over the C++ bindings mirror", flush=True)
    proc = subprocess.run([str(HOST_TEST)], capture_output=True, text=True, timeout=300)
    print(proc.stdout, flush=True)
    if proc.stderr:
        print(proc.stderr, flush=True)
    failed = re.findall(r"^FAIL (.*)$", proc.stdout, re.M)
    assert not failed, failed
    passed = re.findall(r"^PASS (\w+)", proc.stdout, re.M)
    assert passed == EXPECTED, passed
    assert proc.returncode == 0
