"""Write the reference's own kernel golden vectors as fixtures.

Runs the reference's golden generator in its model-free mode,
``scripts/generate_golden.py --kernels-only --device cpu`` (function
``generate_kernel_golden``, scripts/generate_golden.py:166-206), in this
container, and keeps the RMSNorm and SiLU files it writes:

  rmsnorm_input.bin / rmsnorm_weight.bin / rmsnorm_output.bin   [1,1,4096]
  silu_input.bin / silu_output.bin                              [11008]

Each file is raw little-endian fp32 (save_tensor, generate_golden.py:25-32)
holding values computed in torch fp16 on the CPU from torch.manual_seed(42)
draws. The GEMM files it also writes are outside this library's scope and
are deleted. Only the data files are committed; the reference's code is
never copied. Usage (from the repo root):

    python tests/golden/gen_reference_golden.py /root/reference
"""
from __future__ import annotations

import importlib.util
import sys
import tempfile
from pathlib import Path

KEEP = [
    "rmsnorm_input.bin",
    "rmsnorm_weight.bin",
    "rmsnorm_output.bin",
    "silu_input.bin",
    "silu_output.bin",
]


def main(reference_root: str) -> None:
    script = Path(reference_root) / "scripts" / "generate_golden.py"
    spec = importlib.util.spec_from_file_location("ng_reference_generate_golden", script)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    out_dir = Path(__file__).resolve().parent / "reference_kernels"
    out_dir.mkdir(exist_ok=True)
    with tempfile.TemporaryDirectory() as tmp:
        mod.generate_kernel_golden(Path(tmp), device="cpu")
        for name in KEEP:
            (out_dir / name).write_bytes((Path(tmp) / name).read_bytes())
    print(f"wrote {len(KEEP)} fixtures to {out_dir}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
