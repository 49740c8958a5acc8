"""Build libkvq.so (the C-ABI HIP library) in-tree for gfx950.

    python -m llm_kvcache_quantization_amd.build

One hipcc invocation compiles every ``csrc/*.hip`` file for ``--offload-arch=gfx950``
into ``llm_kvcache_quantization_amd/libkvq.so``.  The library links the HIP runtime
by SONAME (``libamdhip64.so.7``).  When PyTorch-ROCm is imported first, the runtime
PyTorch already loaded is reused, so kernels and torch share streams and memory.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libkvq.so"
ARCH = os.environ.get("KVQ_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm at /opt/rocm)")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build_command(out: Path = LIB_PATH) -> list[str]:
    return [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        # packed-fp32 VALU forms are disabled: the code never relies on them
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        *[str(s) for s in sources()],
        "-o", str(out),
    ]


def build(verbose: bool = False) -> Path:
    """Compile libkvq.so; always recompiles.  Returns the library path."""
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = build_command(tmp)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is harmless
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
