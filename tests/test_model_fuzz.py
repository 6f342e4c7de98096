""".qw header fuzz and the threaded file reader, host only (ModelStore.Open, ModelStore.cs:85-127).

ModelStore.Open trusts nothing in the file but the magic; the C-ABI replacement parses the
JSON header by hand, so every corruption must end in an error status (or a valid handle
whose tensors stay inside the file), never in a crash or an out-of-bounds access.  The cases
are seeded mutations of a valid header (byte flips, insertions, deletions, truncations, a
rewritten length field) and hand-made hostile headers (deep nesting, numbers at the int64
limits, offsets and sizes whose sum overflows, unpaired surrogate escapes, NUL bytes).  The
sanitizer builds of the host code (``make -C qauntrunner_amd/csrc sanitize``) run this file
under AddressSanitizer + UndefinedBehaviorSanitizer and under ThreadSanitizer.
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import qauntrunner_amd as qr
from qauntrunner_amd import _lib

ERRORS = {_lib.QR_ERR_INVALID_ARGUMENT, _lib.QR_ERR_OUT_OF_MEMORY}


def _file_bytes(header, data, hlen=None):
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    start = (8 + len(hb) + 63) & ~63
    return (b"QWR1" + struct.pack("<i", len(hb) if hlen is None else hlen) + hb + b"\0" * (start - 8 - len(hb)) +
            bytes(data))


def _valid(n=4):
    tensors = [{"name": f"l{i // 2}.t{i}", "dims": [4, 8], "format": i % 3, "offset": 128 * i, "size": 128}
               for i in range(n)]
    return {"config": {"arch": "llama", "dim": 8}, "tensors": tensors}, np.arange(128 * n, dtype=np.uint8)


def _open_and_use(path):
    """Opens the file; on success walks every tensor (info and a full read) and closes."""
    L = qr.load()
    h = ctypes.c_void_p()
    st = L.qr_model_open(ctypes.byref(h), path.encode())
    if st != _lib.QR_OK:
        assert st in ERRORS, (st, L.qr_last_error())
        assert not h.value and L.qr_last_error()
        return st
    try:
        count = ctypes.c_int()
        assert L.qr_model_tensor_count(h, ctypes.byref(count)) == 0
        size = os.path.getsize(path)
        for i in range(count.value):
            buf = ctypes.create_string_buffer(1 << 17)
            assert L.qr_model_tensor_name(h, i, buf, len(buf)) == 0
            fmt, nd, nbytes = ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
            dims = (ctypes.c_longlong * 64)()
            st = L.qr_model_tensor_info(h, buf.value, ctypes.byref(fmt), ctypes.byref(nd), dims, 64,
                                        ctypes.byref(nbytes))
            assert st in ERRORS | {_lib.QR_OK}
            if st == _lib.QR_OK:
                assert 0 <= nbytes.value <= size
                dst = np.zeros(max(nbytes.value, 1), np.uint8)
                assert L.qr_model_read(h, buf.value, dst.ctypes.data, dst.size) == 0
    finally:
        assert L.qr_model_close(h) == 0
    return _lib.QR_OK


def test_seeded_mutations_of_a_valid_header(tmp_path):
    header, data = _valid()
    base = bytearray(_file_bytes(header, data))
    hend = 8 + len(json.dumps(header).encode())
    rng = np.random.default_rng(2024)
    path = str(tmp_path / "m.qw")
    outcomes = {}
    for case in range(600):
        b = bytearray(base)
        kind = case % 6
        if kind == 0:  # flip bytes of the header text
            for _ in range(int(rng.integers(1, 9))):
                b[int(rng.integers(8, hend))] ^= int(rng.integers(1, 256))
        elif kind == 1:  # truncate anywhere
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 2:  # rewrite the header length
            v = int(rng.choice([0, -1, 1, hend - 9, hend - 7, hend, len(b), 2 ** 31 - 1, -2 ** 31,
                                int(rng.integers(-2 ** 31, 2 ** 31))]))
            b[4:8] = struct.pack("<i", v)
        elif kind == 3:  # insert printable or structural bytes into the header
            at = int(rng.integers(8, hend))
            ins = bytes(rng.choice(list(b'{}[]",:0123456789-eE.\\u tfn\x00'), int(rng.integers(1, 6))))
            b = b[:at] + ins + b[at:]
            b[4:8] = struct.pack("<i", hend - 8 + len(ins))
        elif kind == 4:  # delete a span of the header
            at = int(rng.integers(8, hend - 1))
            n = int(rng.integers(1, 12))
            del b[at:at + n]
            b[4:8] = struct.pack("<i", max(hend - 8 - n, 1))
        else:  # random header bytes of the same length
            b[8:hend] = rng.integers(0, 256, hend - 8, dtype=np.uint8).tobytes()
        with open(path, "wb") as f:
            f.write(bytes(b))
        st = _open_and_use(path)
        outcomes[st] = outcomes.get(st, 0) + 1
    assert outcomes.get(_lib.QR_ERR_INVALID_ARGUMENT, 0) > 100  # most mutations are rejected


HOSTILE = {
    "deep_array": b'{"config": {}, "tensors": ' + b"[" * 100000 + b"]" * 100000 + b"}",
    "deep_object": b'{"config": {}, "tensors": [], "x": ' + b'{"a": ' * 5000 + b"1" + b"}" * 5000 + b"}",
    "int64_max_offset": {"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 0,
                                                    "offset": 2 ** 63 - 1, "size": 1}]},
    "int64_max_size": {"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 0, "offset": 64,
                                                  "size": 2 ** 63 - 1}]},
    "offset_plus_size_overflow": {"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 0,
                                                             "offset": 2 ** 62, "size": 2 ** 62}]},
    "int_beyond_int64": b'{"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 0, '
                        b'"offset": 99999999999999999999999, "size": 4}]}',
    "data_offset_int64_max": {"config": {}, "data_offset": 2 ** 63 - 1,
                              "tensors": [{"name": "a", "dims": [4], "format": 0, "offset": 0, "size": 0}]},
    "data_offset_negative": {"config": {}, "data_offset": -(2 ** 63),
                             "tensors": [{"name": "a", "dims": [4], "format": 0, "offset": 0, "size": 4}]},
    "huge_dims": {"config": {}, "tensors": [{"name": "a", "dims": [2 ** 62, 2 ** 62, 4], "format": 0,
                                             "offset": 0, "size": 4}]},
    "format_beyond_int": {"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 2 ** 40,
                                                     "offset": 0, "size": 4}]},
    "unpaired_surrogate": b'{"config": {}, "tensors": [{"name": "\\ud800\\udfff\\ud800", "dims": [4], '
                          b'"format": 0, "offset": 0, "size": 4}]}',
    "short_unicode_escape": b'{"config": {}, "tensors": [{"name": "\\u12", "dims": [4]}]}',
    "nul_in_number": b'{"config": {}, "tensors": [{"name": "a", "dims": [4\x00], "format": 0, "offset": 0, "size": 4}]}',
    "nul_in_name": b'{"config": {}, "tensors": [{"name": "a\x00b", "dims": [4], "format": 0, "offset": 0, "size": 4}]}',
    "long_name": {"config": {}, "tensors": [{"name": "n" * 100000, "dims": [4], "format": 0, "offset": 0,
                                             "size": 4}]},
    "many_tensors": {"config": {}, "tensors": [{"name": f"t{i}", "dims": [1], "format": 0, "offset": 0,
                                                "size": 1} for i in range(20000)]},
    "exponent_overflow": b'{"config": {}, "tensors": [{"name": "a", "dims": [1e999999], "format": 0}]}',
    "lone_minus": b'{"config": {}, "tensors": [{"name": "a", "dims": [-], "format": 0}]}',
    "unterminated_string": b'{"config": {}, "tensors": [{"name": "abc',
    "backslash_at_end": b'{"config": {}, "tensors": [{"name": "abc\\',
}


@pytest.mark.parametrize("case", sorted(HOSTILE))
def test_hostile_headers(tmp_path, case):
    path = str(tmp_path / f"{case}.qw")
    with open(path, "wb") as f:
        f.write(_file_bytes(HOSTILE[case], np.zeros(256, np.uint8)))
    st = _open_and_use(path)
    if case in ("deep_array", "deep_object", "int64_max_offset", "int64_max_size", "offset_plus_size_overflow",
                "int_beyond_int64", "data_offset_int64_max", "exponent_overflow", "lone_minus",
                "unterminated_string", "backslash_at_end", "short_unicode_escape"):
        assert st == _lib.QR_ERR_INVALID_ARGUMENT, case


def test_threaded_read_of_a_large_tensor(tmp_path, monkeypatch):
    """qr_model_read splits a tensor into chunks read by the prefetch reader threads; every
    byte comes back in place (8 readers over 1 MiB chunks of a 6.5 MiB tensor)."""
    monkeypatch.setenv("QR_PREFETCH_READERS", "8")
    monkeypatch.setenv("QR_PREFETCH_CHUNK_MB", "1")
    rng = np.random.default_rng(77)
    big = rng.integers(0, 256, (13 << 19) + 12345, dtype=np.uint8)
    small = rng.integers(0, 256, 4096, dtype=np.uint8)
    header = {"config": {}, "tensors": [{"name": "small", "dims": [4096], "format": 0, "offset": 0, "size": 4096},
                                        {"name": "big", "dims": [big.size], "format": 0, "offset": 4096,
                                         "size": int(big.size)}]}
    path = str(tmp_path / "big.qw")
    with open(path, "wb") as f:
        f.write(_file_bytes(header, np.concatenate([small, big])))
    L = qr.load()
    h = ctypes.c_void_p()
    assert L.qr_model_open(ctypes.byref(h), path.encode()) == 0
    try:
        for _ in range(3):
            got = np.zeros(big.size, np.uint8)
            assert L.qr_model_read(h, b"big", got.ctypes.data, got.size) == 0
            assert np.array_equal(got, big)
        got = np.zeros(small.size, np.uint8)
        assert L.qr_model_read(h, b"small", got.ctypes.data, got.size) == 0
        assert np.array_equal(got, small)
    finally:
        L.qr_model_close(h)
