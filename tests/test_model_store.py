"""ModelStore (.qw) parsing through the C ABI, host only (ModelStore.cs:45-232).

The round trip follows the reference's own store test (tests/QuantRunner.Tests/
Program.cs:168-215): a Q4_K payload of random bytes and an F32 norm written by the
builder, reopened, sizes and every byte compared.  The rest pins the header rules of
ModelStore.Open (:85-126): the 64-byte-aligned data start, an explicit data_offset, the
errors it raises, and the JSON forms a conforming writer may produce.
"""
import ctypes
import json
import os
import struct

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from qauntrunner_amd import _lib
from tests import qwmodel


def write_raw(path, header, data, pad_to=None, hlen=None):
    hb = header if isinstance(header, bytes) else json.dumps(header).encode()
    start = (8 + len(hb) + 63) & ~63 if pad_to is None else pad_to
    with open(path, "wb") as f:
        f.write(b"QWR1" + struct.pack("<i", len(hb) if hlen is None else hlen) + hb)
        f.write(b"\0" * max(0, start - 8 - len(hb)))
        f.write(data)


def test_store_round_trip_like_the_reference(tmp_path):
    path = str(tmp_path / "rt.qw")
    payload = np.random.default_rng(3).integers(0, 256, 144 * 2 * 256, dtype=np.uint8)  # Q4_K [256, 512]
    norms = (0.5 + np.arange(256, dtype=np.float32)).view(np.uint8)
    b = qr.ModelStoreBuilder(path, {"arch": "llama", "dim": 256, "layers": 1, "heads": 4, "vocab": 256, "ffn": 256})
    b.Plan("tok_emb", (256, 512), 6, payload.size)
    b.Plan("final_norm", (256,), 0, norms.size)
    b.Commit(lambda n: payload if n == "tok_emb" else norms)
    with qr.ModelStore.Open(path) as s:
        assert list(s.Tensors) == ["tok_emb", "final_norm"]
        t = s.Get("tok_emb")
        assert (t.Dims, t.Format, t.SizeBytes, t.NumElements) == ((256, 512), 6, payload.size, 256 * 512)
        assert t.RowBytes() == 288
        assert np.array_equal(s.Read("tok_emb"), payload)
        assert np.array_equal(s.Read("final_norm").view(np.float32), 0.5 + np.arange(256, dtype=np.float32))
        x = np.full(512, 0.25, np.float32)
        assert oracle.matvec(6, s.Read("tok_emb"), 512, x)[7] == oracle.matvec(6, payload, 512, x)[7]
        assert s.Has("final_norm") and not s.Has("nope")
        with pytest.raises(KeyError):
            s.Get("nope")


def test_data_start_is_64_aligned_and_data_offset_wins(tmp_path):
    path = str(tmp_path / "a.qw")
    data = np.arange(200, dtype=np.uint8)
    hdr = {"config": {}, "tensors": [{"name": "a", "dims": [200], "format": 0, "offset": 0, "size": 200}]}
    hb = json.dumps(hdr).encode()
    write_raw(path, hb, data)
    with qr.ModelStore.Open(path) as s:
        assert np.array_equal(s.Read("a"), data)
    # absolute data_offset 300 -> data at 320 (ModelStore.cs:101-104)
    hdr["data_offset"] = 300
    write_raw(path, json.dumps(hdr).encode(), data, pad_to=320)
    with qr.ModelStore.Open(path) as s:
        assert np.array_equal(s.Read("a"), data)
    # the builder's reserved-header form
    b = qr.ModelStoreBuilder(path, {"k": 1}, header_reserve_bytes=1000)
    b.Plan("x", (4, 8), 0, 128)
    b.Commit(lambda n: np.arange(128, dtype=np.uint8))
    raw = open(path, "rb").read()
    head = json.loads(raw[8:8 + struct.unpack("<i", raw[4:8])[0]])
    assert head["data_offset"] == (8 + 1000 + 63) & ~63
    with qr.ModelStore.Open(path) as s:
        assert np.array_equal(s.Read("x"), np.arange(128, dtype=np.uint8))


def test_offsets_are_relative_to_the_data_start(tmp_path):
    path = str(tmp_path / "o.qw")
    data = np.random.default_rng(1).integers(0, 256, 1000, dtype=np.uint8)
    hdr = {"config": {"nested": [1, 2.5e-3, True, None, {"s": "x"}]}, "tensors": [
        {"name": "b", "dims": [10, 10], "format": 0, "offset": 600, "size": 400},
        {"name": "a", "dims": [3], "format": 4, "offset": 0, "size": 600}]}
    write_raw(path, json.dumps(hdr, indent=2).encode(), data)
    with qr.ModelStore.Open(path) as s:
        assert list(s.Tensors) == ["b", "a"]
        assert np.array_equal(s.Read("b"), data[600:]) and np.array_equal(s.Read("a"), data[:600])
        assert s.Get("b").Dims == (10, 10) and s.Get("a").Format == 4


def test_json_escapes_and_repeated_names(tmp_path):
    """A later entry of the same name replaces the earlier one in place, as a C# dictionary
    assignment does (ModelStore.cs:116); escaped names decode to UTF-8."""
    path = str(tmp_path / "e.qw")
    data = np.arange(64, dtype=np.uint8)
    hdr = {"config": {}, "tensors": [
        {"name": "l0.wéq \"x\"", "dims": [8], "format": 0, "offset": 0, "size": 32},
        {"name": "dup", "dims": [4], "format": 0, "offset": 0, "size": 16},
        {"name": "dup", "dims": [8], "format": 0, "offset": 32, "size": 32}]}
    write_raw(path, json.dumps(hdr, ensure_ascii=True).encode(), data)
    with qr.ModelStore.Open(path) as s:
        assert list(s.Tensors) == ["l0.wéq \"x\"", "dup"]
        assert s.Get("dup").Dims == (8,) and np.array_equal(s.Read("dup"), data[32:])
        assert np.array_equal(s.Read("l0.wéq \"x\""), data[:32])


def test_synthetic_model_layout(tmp_path):
    path = str(tmp_path / "m.qw")
    tensors = qwmodel.write(path, layers=2, experts=2, fmt="Q8_0")
    with qr.ModelStore.Open(path) as s:
        assert list(s.Tensors) == list(tensors)
        for name, (code, dims, raw) in tensors.items():
            v = s.Get(name)
            assert (v.Format, v.Dims, v.SizeBytes) == (code, dims, raw.size)
            assert np.array_equal(s.Read(name), raw)


def open_status(path):
    L = qr.load()
    h = ctypes.c_void_p()
    st = L.qr_model_open(ctypes.byref(h), path.encode())
    return st, L.qr_last_error().decode(), h


@pytest.mark.parametrize("case,needle", [
    ("magic", "not a QuantRunner"),
    ("short", "not a QuantRunner"),
    ("hlen_negative", "header length"),
    ("hlen_past_eof", "header length"),
    ("not_json", "not a JSON object"),
    ("trailing", "not a JSON object"),
    ("no_tensors", "tensors array"),
    ("no_config", "config"),
    ("bad_entry", "malformed tensor"),
    ("float_size", "malformed tensor"),
    ("bad_dims", "bad dims"),
    ("past_eof", "past the end"),
    ("data_offset_small", "data_offset"),
])
def test_open_rejects_corrupt_files(tmp_path, case, needle):
    path = str(tmp_path / f"{case}.qw")
    ok = {"config": {}, "tensors": [{"name": "a", "dims": [4], "format": 0, "offset": 0, "size": 16}]}
    data = np.zeros(16, np.uint8)
    if case == "magic":
        write_raw(path, json.dumps(ok).encode(), data)
        with open(path, "r+b") as f:
            f.write(b"QWR2")
    elif case == "short":
        open(path, "wb").write(b"QWR")
    elif case == "hlen_negative":
        write_raw(path, json.dumps(ok).encode(), data, hlen=-5)
    elif case == "hlen_past_eof":
        write_raw(path, json.dumps(ok).encode(), data, hlen=1 << 20)
    elif case == "not_json":
        write_raw(path, b"{config: 1}", data)
    elif case == "trailing":
        write_raw(path, b"[1, 2", data)
    elif case == "no_tensors":
        write_raw(path, json.dumps({"config": {}}).encode(), data)
    elif case == "no_config":
        write_raw(path, json.dumps({"tensors": ok["tensors"]}).encode(), data)
    elif case == "bad_entry":
        write_raw(path, json.dumps({"config": {}, "tensors": [{"name": "a", "dims": [4]}]}).encode(), data)
    elif case == "float_size":
        t = dict(ok["tensors"][0], size=16.5)
        write_raw(path, json.dumps({"config": {}, "tensors": [t]}).encode(), data)
    elif case == "bad_dims":
        t = dict(ok["tensors"][0], dims=[4, -1])
        write_raw(path, json.dumps({"config": {}, "tensors": [t]}).encode(), data)
    elif case == "past_eof":
        t = dict(ok["tensors"][0], offset=8)
        write_raw(path, json.dumps({"config": {}, "tensors": [t]}).encode(), data)
    elif case == "data_offset_small":
        write_raw(path, json.dumps(dict(ok, data_offset=8)).encode(), data)
    st, msg, h = open_status(path)
    assert st == _lib.QR_ERR_INVALID_ARGUMENT and not h.value, (st, msg)
    assert needle in msg, msg


def test_open_missing_file_and_handle_errors(tmp_path):
    st, msg, _ = open_status(str(tmp_path / "absent.qw"))
    assert st == _lib.QR_ERR_INVALID_ARGUMENT and "cannot open" in msg
    with pytest.raises(qr.QrInvalidArgument):
        qr.ModelStore.Open(str(tmp_path / "absent.qw"))
    path = str(tmp_path / "m.qw")
    qwmodel.write(path, layers=1)
    L = qr.load()
    with qr.ModelStore.Open(path) as s:
        small = ctypes.create_string_buffer(4)
        assert L.qr_model_tensor_name(s.handle, 0, small, 4) == _lib.QR_ERR_INVALID_ARGUMENT   # "tok_emb" needs 8
        assert L.qr_model_tensor_name(s.handle, 99, small, 4) == _lib.QR_ERR_INVALID_ARGUMENT
        dims = (ctypes.c_longlong * 1)()
        assert L.qr_model_tensor_info(s.handle, b"l0.wq", None, None, dims, 1, None) == _lib.QR_ERR_INVALID_ARGUMENT
        assert L.qr_model_tensor_info(s.handle, b"none", None, None, None, 0, None) == _lib.QR_ERR_INVALID_ARGUMENT
        buf = np.empty(10, np.uint8)
        assert L.qr_model_read(s.handle, b"l0.wq", buf.ctypes.data_as(ctypes.c_void_p), 10) == \
            _lib.QR_ERR_INVALID_ARGUMENT
        assert L.qr_model_set_prefetch(s.handle, -1) == _lib.QR_ERR_INVALID_ARGUMENT
        # a disabled pipeline makes no device call: Begin returns at once, the counters stay zero
        p = qr.PrefetchPipeline(s, 0)
        assert not p.Enabled
        p.Begin(0)
        p.WaitLayer(0)
        assert (p.BytesStreamed, p.StagedLayers, p.SkippedLayers) == (0, 0, 0)
    assert L.qr_model_close(None) == 0
    assert L.qr_model_begin(None, 0) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_model_acquire(None, b"a", 0, None, ctypes.byref(ctypes.c_void_p())) == _lib.QR_ERR_INVALID_ARGUMENT


def test_layer_bytes_helper_matches_the_reference_filter():
    """PrefetchPipeline.cs:116-129: prefix "l<n>.", names ending in norm/router excluded."""
    t = {"l1.wq": (0, (1,), np.zeros(10)), "l1.attn_norm": (0, (1,), np.zeros(5)), "l1.router": (0, (1,), np.zeros(7)),
         "l10.wq": (0, (1,), np.zeros(100)), "l1.e0.w_up": (0, (1,), np.zeros(3)), "lm_head": (0, (1,), np.zeros(1000))}
    assert qwmodel.layer_bytes(t, 1) == 13
    assert qwmodel.layer_bytes(t, -1) == 1113


def test_dispose_is_idempotent(tmp_path):
    path = str(tmp_path / "x.qw")
    qwmodel.write(path, layers=1, dim=64, ffn=64, vocab=32, heads=2, fmt="Q8_0")
    s = qr.ModelStore.Open(path)
    s.Dispose()
    s.Dispose()   # idempotent
    os.remove(path)


def test_open_handles_are_closed_at_exit(tmp_path):
    """A handle still open when the interpreter exits is closed by the library's atexit hook
    (while the runtime is whole), and finalizers that run during interpreter shutdown do
    nothing: the process exits with status 0."""
    import subprocess
    import sys

    path = str(tmp_path / "exit.qw")
    qwmodel.write(path, layers=1)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import qauntrunner_amd as qr\n"
            "s = qr.ModelStore.Open(%r)\n"
            "keep = [s]\n"  # still referenced when the interpreter finalizes
            "print(len(s.Tensors))\n") % (root, path)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert int(r.stdout.strip()) > 0
