"""Shared helpers for the tests (loading the host-check library, seeds)."""
import ctypes
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
HOSTCHECK = ROOT / "tests" / "native" / "libmkv_hostcheck.so"
GOLDEN = ROOT / "tests" / "golden"

_hc = None


def hostcheck():
    """The g++ build of muserve_amd/csrc/mkv_common.h (built by __graft_entry__.build)."""
    global _hc
    if _hc is None:
        if not HOSTCHECK.exists():
            import __graft_entry__
            __graft_entry__.build_hostcheck()
        lib = ctypes.CDLL(str(HOSTCHECK))
        P, I64, I32, U32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32
        lib.hc_e4m3fn_encode_bits.argtypes = [ctypes.c_uint64, ctypes.c_uint64, P]
        lib.hc_e4m3fn_encode.argtypes = [P, P, I64]
        lib.hc_e4m3fn_decode.argtypes = [P, P, I64]
        lib.hc_bf16_rne.argtypes = [P, P, I64]
        lib.hc_page_hashes.argtypes = [P, I64, I32, P]
        for f in (lib.hc_e4m3fn_encode_bits, lib.hc_e4m3fn_encode, lib.hc_e4m3fn_decode,
                  lib.hc_bf16_rne, lib.hc_page_hashes):
            f.restype = None
        _hc = lib
    return _hc


def np_ptr(a: np.ndarray) -> int:
    return a.ctypes.data
