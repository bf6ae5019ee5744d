"""The kernels' interval masks (probjax_amd/csrc/attn_mods.h) on the CPU.

``row_bounds`` (keys a query row sees) and ``key_bounds`` (rows that see a
key) are checked against the masks' element-wise definitions on random
combinations of causal shift, windows, prefix-LM and sequence lengths, KV and
static lengths, and the row bounds for monotonicity (the tile ranges rely on
it).  The header is compiled for the host only by hipcc.
"""

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


def _hipcc():
    for cand in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    return None


def test_interval_bounds_match_elementwise_masks(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    exe = tmp_path / "mask_bounds_check"
    res = subprocess.run([hipcc, "--cuda-host-only", "-O1", "-std=c++17", str(HERE / "mask_bounds_check.hip"),
                          "-o", str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert run.stdout.startswith("ok ")
    assert int(run.stdout.split()[1]) > 1_000_000
