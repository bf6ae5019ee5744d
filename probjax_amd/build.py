"""Build the gfx950 HIP kernel library ``probjax_amd/_lib/libprobjax_hip.so``.

Compiles every ``csrc/*.hip`` with hipcc for gfx950 only, in parallel, and
links one shared library exporting the C ABI of ``include/probjax_hip.h``.
Run ``python -m probjax_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libprobjax_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # NaN inputs still propagate (through exp2, the row sums and the outputs);
    # this only drops the canonicalising moves the compiler puts around every
    # fmaxf of the row-max reductions.
    "-fno-honor-nans",
    # Packed-fp32 VALU forms are disabled for every kernel of this library.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Extra flags for single sources.  flash_bias_ring.hip: its LDS ring leaves one
# wave per SIMD, and at that occupancy the compiler would put the MFMA
# accumulators in AGPRs and copy every score out of them for the softmax;
# forcing the VGPR form of the MFMAs keeps the scores where the softmax reads
# them (the kernel fits in 256 VGPRs).  flash_wide.hip: the same at one wave
# per SIMD, and worse: with the output accumulators in AGPRs the compiler
# copies all of them to VGPRs at the top of every key tile for the rarely
# taken rescale (128-144 v_accvgpr_read per tile).  In the VGPR form the
# accumulators stay in VGPRs and part of Q^T goes to AGPRs, which the MFMAs
# read directly (latent prefill forward 5.6% faster, the dense-bias forwards
# 4%).  decode.hip: the same copies around the accumulators of the 64-row GQA
# decode and of the fp32 decodes (GQA-8 with 8 query rows 5.7% faster, fp32
# decode 3%; the bf16 C3 / latent decode unchanged).  flash_fwd.hip: the fp32
# forward kernels likewise (7-8.5% faster); its 16-bit kernels use no AGPRs
# and compile to the same code either way.  flash_bwd.hip: the fp32 backward
# kernels (5-6% faster) and the 16-bit ones (1%); its D = 256 dK/dV kernel,
# which the compiler fails on in that form, is built from flash_bwd256.hip in
# the default form.  flash_wide_bwd.hip keeps the default: the VGPR form made
# its latent backward 44% slower.
FILE_FLAGS = {
    "flash_bias_ring.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "flash_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "flash_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "flash_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def _compile(src: Path, obj: Path) -> str:
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{out}")
    return out


def build(verbose: bool = False) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    OUT_DIR.mkdir(exist_ok=True)
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        logs = list(pool.map(_compile, sources, objs))
    if verbose:
        for s, log in zip(sources, logs):
            if log.strip():
                print(f"[{s.name}]\n{log}")
    lib = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
