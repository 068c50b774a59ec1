"""Build libmuserve_kv.so (the gfx950 HIP kernels behind include/mkv.h).

Usage: ``python -m muserve_amd.build``. Compiles every ``csrc/*.hip`` with
hipcc for gfx950 into ``muserve_amd/_build/`` and links the shared library
in-tree at ``muserve_amd/libmuserve_kv.so`` (replaced atomically, so a process
that already mapped the old file keeps a consistent copy).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB_NAME = "libmuserve_kv.so"
LIB_PATH = PKG / LIB_NAME

ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (some forms have given
# wrong results on this hardware). No fast-math anywhere: the fp8 quantiser
# relies on correctly rounded fp32 division. -fno-strict-aliasing: kernels read
# byte buffers and packed records through vector types.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fno-strict-aliasing",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the muserve_amd kernels need ROCm's hipcc")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(
            f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    noise = [ln for ln in res.stderr.splitlines()
             if ln.strip() and "packed-fp32-ops" not in ln and "warning generated" not in ln]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources and link the library; returns its path."""
    cc = hipcc()
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in sources]
    cmds = [[cc, *HIP_FLAGS, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for cmd, fut in [(c, ex.submit(_run, c)) for c in cmds]:
            if verbose:
                print(" ".join(cmd))
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
