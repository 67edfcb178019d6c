"""Build libcachalot_amd.so (gfx950 only) in-tree with hipcc.

    python -m cachalot_amd.build          # compile every csrc/*.hip, link the .so

Flags: ``--offload-arch=gfx950`` only; ``-ffp-contract=off`` so float
operations round exactly as written (the router's bit-exact contract and the
synthetic generator depend on it; fused multiply-adds are written explicitly
where wanted); packed-FP32 instruction selection disabled
(``-target-feature -packed-fp32-ops``).
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
OUT = PKG / "libcachalot_amd.so"
OBJ = PKG / "_build"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file flags.  prefill_affine_mx.hip: matrix-core results in VGPRs, where its
# per-group fold reads them (the other kernels keep their accumulators in AGPRs).
FILE_FLAGS = {"prefill_affine_mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr[-6000:]}")
    return obj


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(srcs)} sources", flush=True)
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
