"""ctypes binding of libmuserve_kv.so (C ABI in include/mkv.h).

The library is loaded after torch, so its HIP runtime references bind to the
runtime torch already mapped: a hipStream_t from torch and a device pointer
from a torch tensor mean the same thing on both sides of the boundary.

Every wrapper here launches asynchronously on the current torch stream of the
tensors' device. Data-dependent faults are reported through a per-owner int32
device word (``DeviceErrors``) that callers check at their sync points.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libmuserve_kv.so")
ABI_VERSION = 1

# device error bits (include/mkv.h)
DEVERR_SLOT = 1
DEVERR_PAGE = 2
DEVERR_TABLE = 4
DEVERR_STATE_SLOT = 8
DEVERR_NEW_PAGE = 16
DEVERR_BM = 32
DEVERR_DUP = 64
_DEVERR_TEXT = {
    DEVERR_SLOT: "slot_mapping entry out of range",
    DEVERR_PAGE: "page id out of range",
    DEVERR_TABLE: "sequence longer than its block table (or inconsistent offsets)",
    DEVERR_STATE_SLOT: "state-pool slot out of range",
    DEVERR_NEW_PAGE: "decode step needed a new page but none was supplied",
    DEVERR_BM: "block manager: malformed request or release of a request not admitted",
    DEVERR_DUP: "an index that must be unique appears more than once",
}

# Default of the opt-in duplicate-index check (PagedKVCache.check_unique,
# StatePool.check_unique): on when MUSERVE_KV_CHECK_UNIQUE is set to anything
# but "" or "0". Off by default: it costs two small launches per guarded call.
CHECK_UNIQUE_DEFAULT = os.environ.get("MUSERVE_KV_CHECK_UNIQUE", "") not in ("", "0")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F32 = ctypes.c_float

# name -> argtypes, in the order of include/mkv.h
SIGNATURES: dict[str, list] = {
    "mkv_version": [],
    "mkv_last_error": [],
    "mkv_append_bf16": [_P, _P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _I32, _I32, _P, _P],
    "mkv_gather_bf16": [_P, _P, _I64, _I64, _P, _I64, _I32, _P, _P, _I32, _I64, _P, _P, _P,
                        _I64, _I32, _I32, _P, _P],
    "mkv_decode_slots": [_P, _P, _I64, _I32, _P, _I32, _I64, _P, _P, _P],
    "mkv_check_unique": [_P, _I32, _I64, _I64, _P, _I64, _P, _P],
    "mkv_step_plan": [_P, _I64, _I32, _I32, _P, _I32, _P, _I32, _I64, _P, _P, _I64, _P, _I64, _I32,
                      _P, _P, _P, _P, _P],
    "mkv_append_fp8": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _I32,
                       _I32, _I32, _P, _P],
    "mkv_gather_dequant_fp8": [_P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _I32,
                               _I64, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P],
    "mkv_copy_blocks": [_P, _I64, _I32, _I64, _I64, _P, _P, _I32, _P, _P],
    "mkv_state_gather": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _I32, _P, _P],
    "mkv_state_scatter": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _I32, _P, _P],
    "mkv_gdn_conv_decode": [_P, _I64, _I32, _I32, _P, _I32, _P, _P, _I32, _P, _P, _P],
    "mkv_gdn_decode_gather": [_P, _I64, _P, _P, _I32, _I32, _I64, _P, _I32, _P, _P, _I32, _P,
                              _P, _P],
    "mkv_pack_blocks": [_P, _I64, _I32, _I64, _I64, _P, _I32, _P, _P, _P],
    "mkv_unpack_blocks": [_P, _I64, _I32, _I64, _I64, _P, _I32, _P, _P, _P],
    "mkv_zero_blocks": [_P, _I64, _I32, _I64, _I64, _P, _I32, _P, _P],
    "mkv_block_hash_sha256": [_P, _P, _P, _I32, _I32, _P, _P, _P],
    "mkv_prefill_attention_bf16": [_P, _P, _P, _I64, _I32, _I32, _I32, _P, _I64, _I32, _P, _P,
                                   _P, _I32, _I64, _I32, _F32, _I32, _I32, _I32, _P, _P, _I64,
                                   _P, _P],
    "mkv_prefill_attention_workspace_bytes": [_I64, _I32, _I32],
    "mkv_check_conversions": [_P, _P],
    "mkv_bm_state_bytes": [_I32],
    "mkv_bm_layout": [_I32, _P],
    "mkv_bm_init": [_P, _I32, _P, _P],
    "mkv_bm_step": [_P, _I32, _P, _I32, _I32, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P, _P,
                    _I64, _P, _P],
    "mkv_bm_step_begin": [_P, _I32, _P, _I32, _I32, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P,
                          _P, _I64, _P, _P],
    "mkv_bm_step_end": [_P, _I32, _P, _I32, _I32, _P, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _P,
                        _P, _I64, _P, _P],
    "mkv_hash_probe": [_P, _I32, _P, _P, _I32, _P, _P, _P, _P],
    "mkv_decode_attention_workspace_bytes": [_I32, _I32, _I32, _I32],
    "mkv_decode_attention_bf16": [_P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _I64, _I32, _P,
                                  _I32, _I32, _F32, _P, _P, _I64, _P, _P],
    "mkv_decode_attention_bf16_noalloc": [_P, _P, _P, _I64, _I32, _I32, _I32, _P, _I64, _I32, _P,
                                          _I32, _I32, _F32, _P, _P, _P],
    "mkv_decode_attention_f16": [_P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _I64, _I32, _P,
                                 _I32, _I32, _F32, _P, _P, _I64, _P, _P],
    "mkv_decode_attention_fp8": [_P, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _P, _I64, _I32,
                                 _P, _I32, _I32, _F32, _P, _P, _I64, _P, _P],
    "mkv_decode_attention_contig": [_P, _P, _P, _I32, _I32, _I32, _I32, _I64, _P, _I32, _I32, _F32,
                                    _P, _P, _I64, _P, _P],
    "mkv_probe_read_pages": [_P, _P, _I32, _I64, _P, _I64, _I32, _I32, _P, _P],
    "mkv_probe_scatter_pages": [_P, _I64, _P, _I64, _I64, _P, _I32, _I32, _P],
    "mkv_probe_fill": [_P, _I64, _P],
}
_INT64_RESULT = {"mkv_bm_state_bytes", "mkv_decode_attention_workspace_bytes",
                 "mkv_prefill_attention_workspace_bytes"}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class MkvError(RuntimeError):
    """A libmuserve_kv entry point returned a non-OK status."""


class MkvDeviceError(RuntimeError):
    """A kernel flagged a data-dependent fault in its device error word."""


def _hip_runtimes() -> list[str]:
    try:
        with open("/proc/self/maps") as f:
            return sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln})
    except OSError:
        return []


def load() -> ctypes.CDLL:
    """Loads (once) and returns the library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built ({LIB_PATH}); build it with "
                "`python -m muserve_amd.build` — there is no fallback path")
        torch.zeros(1)  # make sure torch's HIP runtime is mapped before ours resolves
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = (ctypes.c_char_p if name == "mkv_last_error" else
                          ctypes.c_int64 if name in _INT64_RESULT else ctypes.c_int)
        if lib.mkv_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {lib.mkv_version()} != expected {ABI_VERSION}")
        runtimes = _hip_runtimes()
        if len(runtimes) > 1:
            raise RuntimeError(f"two HIP runtimes are mapped ({runtimes}); load torch first")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Calls an entry point and raises MkvError on a non-OK status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.mkv_last_error().decode(errors="replace")
        raise MkvError(f"{name} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm device; returns it."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"muserve_amd kernels run on a ROCm GPU only; got a tensor on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


# torch's accessor of the current stream's raw handle (what its own kernel
# launchers use): ~0.3 us against ~6 us for current_stream(device).cuda_stream,
# which matters to steps made of many short launches
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The hipStream_t (as an int) of torch's current stream on ``device``."""
    if _raw_stream is not None:
        idx = device.index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream


CONVERSION_COUNTERS = ("fp8_encode_mismatch", "bf16_mismatch", "fp8_decode_mismatch",
                       "div_code_mismatch", "div_quotient_mismatch", "fp32_values", "div_pairs")


def check_conversions(device: torch.device | str = "cuda") -> dict[str, int]:
    """Runs mkv_check_conversions on ``device`` and returns its counters."""
    dev = torch.device(device)
    counts = torch.zeros(len(CONVERSION_COUNTERS), dtype=torch.int64, device=dev)
    call("mkv_check_conversions", counts.data_ptr(), stream_of(dev))
    return dict(zip(CONVERSION_COUNTERS, counts.cpu().tolist()))


class UniqueCheck:
    """Bitmap over the indices [0, limit) for mkv_check_unique; zero between
    calls (each call clears the words it set). Use it on one stream."""

    def __init__(self, device: torch.device, limit: int):
        self.limit = int(limit)
        self.bits = torch.zeros(max(1, (self.limit + 31) // 32), dtype=torch.int32, device=device)

    def run(self, ids: torch.Tensor, err: "DeviceErrors") -> None:
        """Flags (DEVERR_DUP in ``err``) any index of ``ids`` in [0, limit)
        that appears twice; asynchronous on the current stream."""
        if ids.dtype not in (torch.int32, torch.int64) or not ids.is_contiguous():
            raise TypeError("ids must be a contiguous int32 or int64 tensor")
        if ids.numel() == 0:
            return
        call("mkv_check_unique", ids.data_ptr(), ids.element_size(), ids.numel(), self.limit,
             self.bits.data_ptr(), self.bits.numel(), err.ptr(), stream_of(ids.device))


class DeviceErrors:
    """An int32 device word the kernels OR fault bits into."""

    def __init__(self, device: torch.device):
        self.word = torch.zeros(1, dtype=torch.int32, device=device)

    def ptr(self) -> int:
        return self.word.data_ptr()

    def check(self, what: str = "kernel") -> None:
        """Synchronises with the word's stream; raises and clears on any fault."""
        bits = int(self.word.item())
        if bits:
            self.word.zero_()
            text = "; ".join(t for b, t in _DEVERR_TEXT.items() if bits & b) or f"bits {bits:#x}"
            raise MkvDeviceError(f"{what}: device fault: {text}")
