"""Build the HIP library of the sparse-attention path (gfx950) in-tree: dsv41_amd/libdsv41_hip.so.

Each csrc/*.hip file is compiled separately (in parallel) with hipcc for gfx950 and linked into one shared library
with a C ABI (include/dsv41_hip.h).  Packed-fp32 instructions are disabled for all device code."""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parent.parent / "include"
LIB = PKG / "libdsv41_hip.so"
OBJ = PKG.parent / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1", f"-I{INCLUDE}", f"-I{CSRC}"]


def _compile(src: Path, extra=(), tag: str = "") -> Path:
    obj = OBJ / (src.stem + tag + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    return obj


def build(verbose: bool = False, out: Path | None = None, defines=()) -> Path:
    """Compile and link; `out`/`defines` build a variant library (e.g. -DDSV41_TIMING phase timestamps)."""
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    extra = [f"-D{d}" for d in defines]
    tag = "".join("_" + d.lower() for d in defines)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda p: _compile(p, extra, tag), srcs))
    target = Path(out) if out else LIB
    tmp = target.with_suffix(".so.tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, target)
    if verbose:
        print(f"built {target}", file=sys.stderr)
    return target


if __name__ == "__main__":
    build(verbose=True)
