"""Host pieces of the qualification records (libwafer_hip_seam.so, no GPU):
SHA-256 against hashlib (FIPS 180-4 test vectors and random lengths around
the block boundaries) and the canonical JSON printer/parser against Python's
json with sorted keys and compact separators."""
import ctypes
import hashlib
import json
import pathlib

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SEAM = ROOT / "vibe_compiler_amd" / "lib" / "libwafer_hip_seam.so"


@pytest.fixture(scope="module")
def L():
    if not SEAM.exists():
        pytest.skip("seam library not built")
    lib = ctypes.CDLL(str(SEAM))
    lib.wafer_sha256_digest.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_char_p]
    lib.wafer_canonical_json.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    return lib


def digest(L, data: bytes) -> str:
    out = ctypes.create_string_buffer(72)
    buf = ctypes.create_string_buffer(data, len(data))
    L.wafer_sha256_digest(buf, len(data), out)
    return out.value.decode()


def test_sha256_vectors(L):
    # FIPS 180-4 examples ("abc", the two-block message) and the empty string
    assert digest(L, b"abc") == "sha256:ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert digest(L, b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") == \
        "sha256:248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"
    assert digest(L, b"") == "sha256:e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"
    rng = np.random.default_rng(0)
    for n in list(range(0, 130)) + [1000, 4095, 4096, 65537]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert digest(L, data) == "sha256:" + hashlib.sha256(data).hexdigest(), n


def canon(L, text: str):
    out = ctypes.create_string_buffer(1 << 16)
    rc = L.wafer_canonical_json(text.encode(), out, 1 << 16)
    return rc, out.value.decode()


def test_canonical_json_matches_python(L):
    docs = [
        {"b": 1, "a": [3, -2, {"z": None, "y": True, "x": False}], "c": "s\"q\\\n"},
        {"schema": "wafer-hip-qualification-record", "n": 9223372036854775807, "m": -9223372036854775807, "e": {}},
        [],
        {"nested": [[[]], [{}], "\u0001"]},
    ]
    for d in docs:
        text = json.dumps(d, indent=2)
        rc, got = canon(L, text)
        assert rc == 0
        assert got == json.dumps(d, sort_keys=True, separators=(",", ":")) + "\n"
        assert canon(L, got) == (0, got)  # idempotent


def test_json_rejections(L):
    for bad in ['{"a":1,"a":2}', '{"a":1.5}', '{"a":1e3}', '{"a":', '[1,]', '{"a" 1}', '"unterminated',
                '{"a":1} x', '{"a":"\\u00e9"}', '{"a":18446744073709551616}']:
        rc, msg = canon(L, bad)
        assert rc == -1, bad
        assert msg.startswith("invalid JSON"), msg
