"""CPU check of the one-token fp8 x fp4 gate/up kernel's LDS layout
(gate_up_fp4_kernel, inferno_amd/csrc/decode_mfma.hpp): region bounds,
pairwise disjointness, alignment, each wavefront's LDS-DMA area and single
ownership of every shared-down output row, over every instantiated shape.
The checker (tests/lds_layout_check.hip) is built with hipcc as a host
program against the kernel's own layout function; it makes no GPU call."""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.mark.parametrize("cus", [256, 304, 80])
def test_gate_up_fp4_lds_layout(tmp_path, cus):
    if not (Path(HIPCC).exists() or shutil.which(HIPCC)):
        pytest.skip("hipcc not found")
    exe = tmp_path / "ldscheck"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O1", "-std=c++17", f"-I{ROOT / 'include'}",
                    f"-I{ROOT / 'inferno_amd' / 'csrc'}", str(ROOT / "tests" / "lds_layout_check.hip"),
                    "-o", str(exe)], check=True, capture_output=True, text=True)
    r = subprocess.run([str(exe), str(cus)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr + r.stdout[-2000:]
    last = r.stdout.strip().splitlines()[-1]
    assert last.startswith("OK ") and int(last.split()[1]) >= 40, last
