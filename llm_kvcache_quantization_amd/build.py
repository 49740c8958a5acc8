"""Build libkvq.so (the C-ABI HIP library) in-tree for gfx950.

    python -m llm_kvcache_quantization_amd.build

Every ``csrc/*.hip`` file is compiled for ``--offload-arch=gfx950`` by its own hipcc process
(in parallel, into a temporary directory), and the objects are linked into
``llm_kvcache_quantization_amd/libkvq.so``.  The library links the HIP runtime
by SONAME (``libamdhip64.so.7``).  When PyTorch-ROCm is imported first, the runtime
PyTorch already loaded is reused, so kernels and torch share streams and memory.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
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


# packed-fp32 VALU forms are disabled: the code never relies on them
_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def compile_command(src: Path, obj: Path) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", *_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
            str(src), "-o", str(obj)]


def link_command(objs: list[Path], out: Path = LIB_PATH) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(o) for o in objs],
            "-o", str(out)]


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; that is harmless
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile libkvq.so; always recompiles.  Returns the library path."""
    srcs = sources()
    jobs = jobs or max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="kvq_build_") as d:
        objs = [Path(d) / (s.stem + ".o") for s in srcs]
        with ThreadPoolExecutor(max_workers=jobs) as ex:
            errs = list(ex.map(lambda so: _run(compile_command(*so)), zip(srcs, objs)))
        errs.append(_run(link_command(objs, tmp)))
    if verbose:
        for e in errs:
            if e.strip():
                print(e, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
