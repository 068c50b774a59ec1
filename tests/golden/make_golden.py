"""Writes the golden fixtures of this directory.

* reference_known_answers.json — the assertions of the reference's only
  KV-path test, muserve/scripts/test_kv_cache.py (alloc/free counts :25-55,
  exact write/read :58-84, SequenceKVState paging :87-111), as data.
* sha256_fips.json — the SHA-256 example vectors of FIPS 180-2 Appendix B
  and the NIST example set (message -> hex digest).
* fp8_e4m3fn_special.json — hand-derived e4m3fn codes for values where an
  RNE encoder is easy to get wrong (signed zero, ties, subnormal edges, the
  448/464/480 boundary), each worked out from the OCP definition.

Run from the repository root: python tests/golden/make_golden.py
"""
import json
import struct
from pathlib import Path

HERE = Path(__file__).resolve().parent


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def next_f32(x: float) -> float:
    (u,) = struct.unpack("<I", struct.pack("<f", x))
    return struct.unpack("<f", struct.pack("<I", u + 1))[0]


known = {
    "alloc_free": {
        "source": "muserve/scripts/test_kv_cache.py:25-55",
        "num_pages": 2000,
        "steps": [
            {"op": "alloc", "n": 1000, "returned": 1000, "free_after": 1000},
            {"op": "free_first_of_last_alloc", "n": 500, "free_after": 1500},
            {"op": "alloc", "n": 600, "returned": 600, "free_after": 900},
            {"op": "alloc_oom", "n": 10000, "raises": "RuntimeError"},
        ],
    },
    "write_read": {
        "source": "muserve/scripts/test_kv_cache.py:58-84",
        "num_pages": 100, "layer": 0, "slot": 0, "max_abs_err": 0.0,
    },
    "sequence_state": {
        "source": "muserve/scripts/test_kv_cache.py:87-111",
        "num_pages": 100, "tokens": 33, "pages_used": 3, "seq_len": 33,
        "last_page_slot": 0, "table_width": 16, "unused_index": 3, "unused_value": 0,
    },
}

fips = [
    {"msg_ascii": "abc",
     "sha256": "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"},
    {"msg_ascii": "",
     "sha256": "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"},
    {"msg_ascii": "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
     "sha256": "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"},
    {"msg_ascii": "abcdefghbcdefghicdefghijdefghijkefghijklfghijklmghijklmnhijklmno"
                  "ijklmnopjklmnopqklmnopqrlmnopqrsmnopqrstnopqrstu",
     "sha256": "cf5b16a778af8380036ce59e7b0492370b249b11e8f07a51afac45037afee9d1"},
    {"msg_ascii": "a", "repeat": 1000000,
     "sha256": "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"},
]

fp8 = [
    {"x": 0.0, "code": 0x00, "why": "+0"},
    {"x": -0.0, "code": 0x80, "why": "-0 keeps its sign"},
    {"x": 1.0, "code": 0x38, "why": "exponent field 7 = bias"},
    {"x": -1.0, "code": 0xB8, "why": "sign bit"},
    {"x": 1.0625, "code": 0x38, "why": "tie 1.0|1.125 -> even mantissa 0"},
    {"x": 1.1875, "code": 0x3A, "why": "tie 1.125|1.25 -> even mantissa 2"},
    {"x": 448.0, "code": 0x7E, "why": "largest finite"},
    {"x": -448.0, "code": 0xFE, "why": "largest finite, negative"},
    {"x": 464.0, "code": 0x7E, "why": "tie 448|480 -> even (448)"},
    {"x": next_f32(464.0), "code": 0x7F, "why": "rounds to 480: NaN (non-saturating cast)"},
    {"x": 2.0 ** -6, "code": 0x08, "why": "smallest normal"},
    {"x": 2.0 ** -9, "code": 0x01, "why": "smallest subnormal"},
    {"x": 2.0 ** -10, "code": 0x00, "why": "tie 0|2^-9 -> even (0)"},
    {"x": next_f32(2.0 ** -10), "code": 0x01, "why": "just above half the smallest subnormal"},
    {"x": 1.5 * 2.0 ** -9, "code": 0x02, "why": "tie 1|2 subnormal -> 2"},
    {"x": 2.5 * 2.0 ** -9, "code": 0x02, "why": "tie 2|3 subnormal -> 2"},
    {"x": 7.5 * 2.0 ** -9, "code": 0x08, "why": "tie 7*2^-9|2^-6 -> 2^-6 (code 8)"},
    {"x": -(2.0 ** -12), "code": 0x80, "why": "negative underflow -> -0"},
    {"x": 240.0, "code": 0x77, "why": "1.875*2^7"},
    {"x": 0.333984375, "code": 0x2B, "why": "1.3359375*2^-2 -> nearest 1.375*2^-2"},
]
for e in fp8:
    e["x"] = f32(e["x"])

(HERE / "reference_known_answers.json").write_text(json.dumps(known, indent=1) + "\n")
(HERE / "sha256_fips.json").write_text(json.dumps(fips, indent=1) + "\n")
(HERE / "fp8_e4m3fn_special.json").write_text(json.dumps(fp8, indent=1) + "\n")
print("wrote", [p.name for p in sorted(HERE.glob("*.json"))])
