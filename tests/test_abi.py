"""The C ABI: header, ctypes bindings and exported symbols agree; argument
errors come back as status codes without touching a GPU."""
import ctypes
import re

import pytest

from muserve_amd import _lib
from tests.helpers import ROOT

HEADER = ROOT / "include" / "mkv.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(mkv_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_bound_functions():
    assert sorted(declared()) == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared():
        assert hasattr(lib, name), name


def test_abi_version():
    assert _lib.load().mkv_version() == _lib.ABI_VERSION


def _rc(name, *args):
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.mkv_last_error().decode()


FAKE = 1 << 20  # an aligned non-null address; argument checks fail before any use


def test_bad_row_bytes_is_an_alignment_error():
    rc, msg = _rc("mkv_append_bf16", FAKE, FAKE, 0, 16, FAKE, FAKE, 0, 32, FAKE, 1, 1, 17, FAKE,
                  None)
    assert rc == -2 and "row_bytes 17" in msg


def test_unsupported_gather_row_size():
    rc, msg = _rc("mkv_gather_bf16", FAKE, FAKE, 0, 4, FAKE, 4, 4, FAKE, None, 1, 16, None, FAKE,
                  FAKE, 0, 1, 96, FAKE, None)
    assert rc == -3 and "row_bytes 96" in msg


def test_fp8_head_dim_must_be_256():
    rc, msg = _rc("mkv_append_fp8", FAKE, FAKE, FAKE, FAKE, 0, 0, 16, FAKE, FAKE, 0, 256, FAKE, 1,
                  1, 1, 128, FAKE, None)
    assert rc == -3 and "head_dim 128" in msg


def test_hash_token_width():
    rc, msg = _rc("mkv_block_hash_sha256", FAKE, FAKE, FAKE, 1, 3, FAKE, FAKE, None)
    assert rc == -3 and "token_bytes 3" in msg


def test_null_pointer_is_invalid():
    rc, msg = _rc("mkv_state_gather", None, 16, None, None, 0, None, 4, FAKE, 2, FAKE, None)
    assert rc == -1 and "null pointer" in msg


def test_empty_calls_are_no_ops():
    assert _rc("mkv_append_bf16", None, None, 0, 0, None, None, 0, 0, None, 0, 1, 512, None,
               None)[0] == 0
    assert _rc("mkv_copy_blocks", None, 0, 2, 4, 8192, None, None, 0, None, None)[0] == 0


def test_probe_arguments():
    rc, msg = _rc("mkv_probe_read_pages", FAKE, FAKE, 1000, 4, FAKE, 4, 0, 1, FAKE, None)
    assert rc == -3 and "page_bytes must be 4096 or 8192" in msg
    rc, msg = _rc("mkv_probe_scatter_pages", FAKE, 8192, FAKE, 4096, 1, FAKE, 2, 1, None)
    assert rc == -1 and "shorter than its pages" in msg
    rc, msg = _rc("mkv_probe_fill", FAKE, 100, None)
    assert rc == -1 and "multiple of 4096" in msg
    assert _rc("mkv_probe_read_pages", None, None, 8192, 0, None, 0, 1, 0, None, None)[0] == 0
    assert _rc("mkv_probe_fill", None, 0, None)[0] == 0


def test_call_raises_with_message():
    with pytest.raises(_lib.MkvError, match="token_bytes 3"):
        _lib.call("mkv_block_hash_sha256", FAKE, FAKE, FAKE, 1, 3, FAKE, FAKE, None)


def test_check_unique_arguments():
    rc, msg = _rc("mkv_check_unique", FAKE, 2, 4, 16, FAKE, 1, FAKE, None)
    assert rc == -1 and "id_bytes 2" in msg
    rc, msg = _rc("mkv_check_unique", FAKE, 8, 4, 100, FAKE, 3, FAKE, None)
    assert rc == -1 and "4 needed" in msg
    assert _rc("mkv_check_unique", None, 8, 0, 100, None, 0, None, None)[0] == 0


def test_noalloc_attention_rejects_an_unsupported_shape():
    # batch x KV heads above 4096: rejected on the host before the scratch
    # lookup or any launch, so fake pointers are never used
    rc, msg = _rc("mkv_decode_attention_bf16_noalloc", FAKE, FAKE, FAKE, 16, 1, 8, 256, FAKE, 1, 1,
                  FAKE, 8192, 2048, 0.0625, FAKE, FAKE, None)
    assert rc == -3 and "unsupported shape" in msg


def test_attention_workspace_of_an_unsupported_shape():
    lib = _lib.load()
    assert lib.mkv_decode_attention_workspace_bytes(4097, 1, 4, 1024) == -1  # too many pairs
    assert lib.mkv_decode_attention_workspace_bytes(8, 1, 3, 1024) == -1     # G = 3
