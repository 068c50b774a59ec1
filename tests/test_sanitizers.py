"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU only).

* The shared arithmetic of muserve_amd/csrc/mkv_common.h (the fp8 encoder and
  decoder, bf16 rounding, the SHA-256 page chain, the quantiser's divide) is
  built by g++ with both sanitizers and run on boundary values and samples.
* The library's host side (every entry point's argument checks, error
  messages, the block manager's layout and the attention workspace sizing) is
  built by hipcc with the sanitizers on the host pass only (``-Xarch_host``;
  the gfx950 code is built as usual) and driven with rejected arguments, so
  no call reaches the GPU.

Any sanitizer report aborts the driver (halt_on_error), which fails the test.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

from tests.helpers import ROOT

NATIVE = ROOT / "tests" / "native"
OUT = NATIVE / "_asan"
CSRC = ROOT / "muserve_amd" / "csrc"
INCLUDE = ROOT / "include"
HIPCC = "/opt/rocm/bin/hipcc"
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


def _run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    assert res.returncode == 0, f"{' '.join(map(str, cmd))}\n{res.stdout}\n{res.stderr}"
    return res


def _check_clean(res):
    text = res.stdout + res.stderr
    assert "AddressSanitizer" not in text and "runtime error" not in text, text


def test_shared_arithmetic_under_sanitizers():
    OUT.mkdir(exist_ok=True)
    exe = OUT / "hostcheck_sanitize"
    _run(["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined",
          "-fno-sanitize-recover=all", f"-I{CSRC}", f"-I{NATIVE}",
          str(NATIVE / "hostcheck_sanitize_main.cpp"), "-o", str(exe)])
    res = _run([str(exe)], env=ENV, timeout=300)
    _check_clean(res)
    assert "0 failures" in res.stdout


@pytest.mark.skipif(not Path(HIPCC).exists() or shutil.which("g++") is None,
                    reason="needs ROCm's hipcc and g++")
def test_entry_point_argument_checks_under_sanitizers():
    OUT.mkdir(exist_ok=True)
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             f"-I{INCLUDE}", f"-I{CSRC}"]
    procs, objs = [], []
    for src in sorted(CSRC.glob("*.hip")):
        obj = OUT / (src.stem + ".o")
        objs.append(obj)
        procs.append(subprocess.Popen([HIPCC, *flags, "-c", str(src), "-o", str(obj)],
                                      stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
    for p in procs:
        out, err = p.communicate()
        assert p.returncode == 0, err
    driver = OUT / "abi_sanitize_main.o"
    _run(["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined",
          f"-I{INCLUDE}", "-c", str(NATIVE / "abi_sanitize_main.cpp"), "-o", str(driver)])
    exe = OUT / "abi_sanitize"
    _run([HIPCC, "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address",
          "-Xarch_host", "-fsanitize=undefined", str(driver), *map(str, objs), "-o", str(exe)])
    res = _run([str(exe)], env=ENV, timeout=300)
    _check_clean(res)
    assert "0 failures" in res.stdout
