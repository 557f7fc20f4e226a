"""The quantizer's reciprocal-and-FMA division (nanochat_amd/csrc/nc_row.h: quant_code) against the plain division,
by tests/quant_division_check.c: every finite bf16 x with |x| <= amax against a strided sample of every bf16 amax
(2 of 64 residues; the full run, every amax, is in the C file's header: 1,065,402,240 pairs, no differing code).
The GPU tests then pin the kernels' codes against the oracle's division (tests/test_gpu_append.py)."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).parent / "quant_division_check.c"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
@pytest.mark.parametrize("part", [0, 37])
def test_reciprocal_division_gives_the_division_codes(tmp_path, part):
    exe = tmp_path / "check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    out = subprocess.run([str(exe), str(part), "64"], capture_output=True, text=True, check=False)
    checked, differ = map(int, out.stdout.split()[-2:])
    assert checked > 10_000_000 and differ == 0, out.stdout
