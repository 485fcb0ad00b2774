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

Every kernel must run without scratch memory: the build reads the compiler's
resource-usage remarks and fails if any kernel has a nonzero ``ScratchSize``.
Several kernels wait on hand-counted vector-memory counts (``s_waitcnt vmcnt``)
that hold only while no compiler-inserted scratch traffic shares the counter,
and a spill would also cost the register budget the designs are sized for.

Usage: ``python oxr-inference_amd/build.py`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import re
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


_NAME = re.compile(r"remark: Function Name: (\S+)")
_SCRATCH = re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")


def scratch_users(remarks: str) -> list[tuple[str, int]]:
    """(kernel, bytes per lane) for every kernel whose resource-usage remark reports scratch."""
    users, name = [], None
    for line in remarks.splitlines():
        if m := _NAME.search(line):
            name = m.group(1)
        elif (m := _SCRATCH.search(line)) and name is not None and int(m.group(1)) > 0:
            users.append((name, int(m.group(1))))
    return users


def _compile(source: Path) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-Rpass-analysis=kernel-resource-usage", "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{' '.join(cmd)}\n{proc.stdout}{proc.stderr}")
    users = scratch_users(proc.stderr)
    if users:
        obj.unlink(missing_ok=True)
        listing = "\n".join(f"  {name}: {size} bytes/lane" for name, size in users)
        raise RuntimeError(f"{source.name}: kernels use scratch memory (register spills), not allowed:\n{listing}")
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
