"""Build recipe for libglm53_hip.so (gfx950 HIP kernels behind include/glm53.h).

`python build_lib.py` or `build_lib.build()` compiles every csrc/*.hip with
hipcc for --offload-arch=gfx950 into this directory.  The library is
built in-tree so it travels with the source tree; nothing is installed.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
LIB_NAME = "libglm53_hip.so"
SOURCES = ["store_int8.hip", "moe_align.hip", "sparse_mla.hip", "moe_w4a16.hip", "indexer.hip", "stream_probe.hip"]

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
# -ffp-contract=off: every fp32 rounding point is the one the source writes.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-ffp-contract=off",
    # keep MFMA accumulators in VGPRs (no AGPR copies around VALU rescales)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # the leading 16 dwords of scalar kernel arguments arrive in SGPRs at
    # wave launch instead of through the first scalar loads (kernels whose
    # arguments are one struct keep loading them; code objects carry the
    # fallback loads for firmware without preloading)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    out = HERE / LIB_NAME
    tmp = HERE / (LIB_NAME + ".tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, *(extra_flags or []), f"-I{ROOT / 'include'}", f"-I{HERE / 'csrc'}",
           *[str(HERE / "csrc" / s) for s in SOURCES], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
