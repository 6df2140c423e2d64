"""Build libgnf4_hip.so in-tree for gfx950 with hipcc.

``python build.py`` (or ``build()``) compiles the HIP sources in csrc/ (the
grouped GEMM kernels and the routing kernels) into ``libgnf4_hip.so`` next to
this file, and the measurement kernels bench.py times against
(``csrc/gnf4_floor.hip``) into ``libgnf4_floor.so``. It always recompiles: the library must
track its source, and the GPU box only ever loads the prebuilt file.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRCS = [HERE / "csrc" / "gnf4_hip.hip", HERE / "csrc" / "gnf4_route.hip"]
OUT = HERE / "libgnf4_hip.so"
FLOOR_SRCS = [HERE / "csrc" / "gnf4_floor.hip"]
FLOOR_OUT = HERE / "libgnf4_floor.so"
ARCH = os.environ.get("GNF4_HIP_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32 for
# ordinary float code (this build targets boxes where those forms are avoided).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-ffp-contract=off", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(srcs, out: Path, verbose: bool) -> Path:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *(str(p) for p in srcs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed ({r.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    _compile(FLOOR_SRCS, FLOOR_OUT, verbose)
    return _compile(SRCS, OUT, verbose)


if __name__ == "__main__":
    print(build(verbose=True))
