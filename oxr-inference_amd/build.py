"""Build the gfx950 HIP library ``liboxr_verify.so`` in-tree.

Every ``csrc/*.hip`` file is compiled to an object with hipcc for gfx950 and the
objects are linked into one shared library next to this file.  The library
exports only the ``extern "C"`` entry points declared in ``include/oxr_verify.h``.

Flags that matter for results:

- ``-ffp-contract=off``: no fused multiply-add where the reference rounds a
  product and a sum separately.
- ``-fhip-fp32-correctly-rounded-divide-sqrt``: fp32 ``/`` and ``sqrtf`` are
  correctly rounded (the RMSNorm ``rsqrt`` is ``1 / sqrt``).
- ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32 VALU
  instructions (``v_pk_*_f32``), which have given intermittently wrong results
  on this machine pool.

Usage: ``python oxr-inference_amd/build.py`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = REPO_DIR / "_build"
LIB_NAME = "liboxr_verify.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{REPO_DIR / 'include'}",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def _compile(source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link ``liboxr_verify.so``; return its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(workers, 1)) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
