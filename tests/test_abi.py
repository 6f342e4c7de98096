"""C-ABI checks that need no GPU: the library loads, exports every entry point the
header declares, and rejects invalid arguments before touching a device."""
import ctypes
import re

import pytest

import qauntrunner_amd as qr
from qauntrunner_amd import _lib


def declared_functions():
    text = open(_lib.HEADER_PATH).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\s*\*)\s+(qr_\w+)\s*\(", text, re.M)))


def test_header_declares_the_binding_table():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_version_and_status_names():
    L = qr.load()
    assert L.qr_abi_version() == 1
    assert L.qr_status_name(0) == b"QR_OK"
    assert L.qr_status_name(-2) == b"QR_ERR_OUT_OF_RANGE"
    assert L.qr_status_name(-5) == b"QR_ERR_NOT_RESIDENT"
    assert L.qr_status_name(-99) == b"QR_ERR_UNKNOWN"


@pytest.mark.parametrize("args,needle", [
    ((0, 8, 2, 64, 512, 0, 1), "layers"),
    ((1, 2, 4, 64, 512, 0, 1), "kv_heads"),
    ((1, 8, 2, 0, 512, 0, 1), "head_dim"),
    ((1, 8, 2, -3, 512, 0, 1), "head_dim"),
    ((1, 8, 2, 513, 512, 0, 1), "head_dim"),   # any head size from 1 to 512
    ((1, 8, 2, 64, 0, 0, 1), "max_seq"),
    ((1, 8, 2, 64, 512, 7, 1), "dtype"),
    ((1, 8, 2, 64, 512, 0, 0), "max_batch"),
])
def test_kv_create_validates_before_device(args, needle):
    L = qr.load()
    h = ctypes.c_void_p()
    st = L.qr_kv_create(ctypes.byref(h), *args)
    assert st == _lib.QR_ERR_INVALID_ARGUMENT and not h.value
    assert needle in L.qr_last_error().decode()


@pytest.mark.parametrize("args", [(0, 512, 64, 100, 2), (1, 0, 64, 100, 2), (1, 2048, 64, 100, 2), (1, 512, -1, 100, 2),
                                  (1, 512, 64, 0, 2), (1, 512, 64, 100, 9)])
def test_mla_create_validates_before_device(args):
    L = qr.load()
    h = ctypes.c_void_p()
    assert L.qr_mla_create(ctypes.byref(h), *args) == _lib.QR_ERR_INVALID_ARGUMENT and not h.value


@pytest.mark.parametrize("latent", [0, 1281, -5])
def test_mla_create_latent_validates_before_device(latent):
    L = qr.load()
    h = ctypes.c_void_p()
    assert L.qr_mla_create_latent(ctypes.byref(h), 1, latent, 100, 2) == _lib.QR_ERR_INVALID_ARGUMENT
    assert not h.value and "latent_dim" in L.qr_last_error().decode()


def test_null_handles_are_rejected():
    L = qr.load()
    out = ctypes.c_int()
    assert L.qr_kv_seq_len(None, 0, ctypes.byref(out)) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_attention(None, 0, 0, 0, None, None, 1.0) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_attention(None, 0, 0, 1, None, None, 1.0, None) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_set_rope(None, 64) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_append_rope_step_dev(None, 0, 0, None, None, None, None, 1e4, None) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_attention_step_dev(None, 1, None, 0, None, None, None, 1.0, None) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_append_rope_chunk_step_dev(None, 0, 0, 4, None, None, None, None, 1e4, None) == \
        _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_attention_chunk_step_dev(None, 0, 0, 4, None, None, 0, None, 1.0, None) == \
        _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_append_step_dev(None, 0, 1, None, None, 0, None) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_attention_step_dev(None, 0, None, 8, None, None, 1.0, None, None) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_attend_absorbed_step_dev(None, 0, None, 8, 128, 128, None, None, 1, None, None) == \
        _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_kv_destroy(None) == 0 and L.qr_mla_destroy(None) == 0
    assert "null" in L.qr_last_error().decode() or L.qr_last_error() == b""


def test_status_maps_to_python_exceptions():
    with pytest.raises(qr.QrInvalidArgument):
        qr.PagedKvCache(1, 8, 2, 600, 512)  # head_dim above 512
    assert issubclass(qr.QrOutOfRange, IndexError) and issubclass(qr.QrNotResident, LookupError)


def test_weight_row_bytes_match_the_oracle():
    """Dtypes.cs:38-50 block specs through the C ABI, for every decoded format."""
    from oracle import oracle
    from qauntrunner_amd import weights

    for name, code in _lib.FORMATS.items():
        for cols in (256, 512, 1024):
            assert weights.row_bytes(code, cols) == oracle.row_bytes(code, cols), (name, cols)
    for fmt, cols in ((5, 256), (3, 48), (6, 128), (99, 8)):
        with pytest.raises(qr.QrInvalidArgument):
            weights.row_bytes(fmt, cols)


def test_projection_arguments_validate_before_device():
    L = qr.load()
    null = ctypes.c_void_p()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails validation first
    assert L.qr_mla_q_absorb_dev(null, 2, 8, 128, 64, 128, 512, 1, fake, fake, null) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_q_absorb_dev(fake, 5, 8, 128, 64, 128, 512, 1, fake, fake, null) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_wuv_dev(fake, 2, 8, 128, 128, 500, 1, fake, fake, null) == _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_wuv_dev(ctypes.c_void_p(0x1002), 2, 8, 128, 128, 512, 1, fake, fake, null) == \
        _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_mla_attend_absorbed(null, 0, 0, 8, 128, 128, fake, fake, fake) == _lib.QR_ERR_INVALID_ARGUMENT
    h = ctypes.c_void_p()
    assert L.qr_weight_create(ctypes.byref(h), 4, 4, 48, fake) == _lib.QR_ERR_INVALID_ARGUMENT and not h.value


def test_matvec_group_arguments_validate_before_device():
    L = qr.load()
    null = ctypes.c_void_p()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced
    ws = (ctypes.c_void_p * 5)(*([0x1000] * 5))
    ys = (ctypes.c_void_p * 5)(*([0x2000] * 5))
    rows = (ctypes.c_longlong * 5)(*([64] * 5))
    err = _lib.QR_ERR_INVALID_ARGUMENT
    assert L.qr_matvec_group_dev(0, ws, rows, 1, 256, 1, fake, ys, null) == err        # empty group
    assert L.qr_matvec_group_dev(5, ws, rows, 1, 256, 1, fake, ys, null) == err        # more than 4
    assert L.qr_matvec_group_dev(2, null, rows, 1, 256, 1, fake, ys, null) == err      # null arrays
    assert L.qr_matvec_group_dev(2, ws, null, 1, 256, 1, fake, ys, null) == err
    assert L.qr_matvec_group_dev(2, ws, rows, 1, 250, 1, fake, ys, null) == err        # cols not a multiple of 8
    bad = (ctypes.c_void_p * 2)(0x1000, 0x1008)
    assert L.qr_matvec_group_dev(2, bad, rows, 1, 256, 1, fake, ys, null) == err       # misaligned weight
    neg = (ctypes.c_longlong * 2)(64, -1)
    assert L.qr_matvec_group_dev(2, ws, neg, 1, 256, 1, fake, ys, null) == err
    assert L.qr_matvec_group_dev(2, ws, rows, 1, 256, 1, ctypes.c_void_p(0x1004), ys, null) == err  # x alignment


class _FakeTensor:
    """Just enough of a torch tensor for the device-argument checks."""

    def __init__(self, numel, dtype="torch.float32", cuda=True, contiguous=True):
        self._n, self.dtype, self.is_cuda, self._c = numel, dtype, cuda, contiguous

    def numel(self):
        return self._n

    def is_contiguous(self):
        return self._c

    def data_ptr(self):
        return 0x1000


def test_device_tensor_arguments_are_checked_on_the_host():
    from qauntrunner_amd.caches import _dev_tensor

    assert _dev_tensor(_FakeTensor(8), 8, _lib.DTYPE_F32, "q").value == 0x1000
    assert _dev_tensor(_FakeTensor(8, "torch.int16"), 8, _lib.DTYPE_F16, "k").value == 0x1000
    assert _dev_tensor(_FakeTensor(8, "torch.bfloat16"), 8, _lib.DTYPE_BF16, "k").value == 0x1000
    assert _dev_tensor(None, 8, _lib.DTYPE_F32, "q_rope", allow_none=True).value is None
    for t, code in ((_FakeTensor(7), _lib.DTYPE_F32),                       # short
                    (_FakeTensor(8, cuda=False), _lib.DTYPE_F32),           # host tensor
                    (_FakeTensor(8, contiguous=False), _lib.DTYPE_F32),     # strided view
                    (_FakeTensor(8, "torch.float16"), _lib.DTYPE_F32),      # wrong element type
                    (_FakeTensor(8, "torch.float16"), _lib.DTYPE_BF16),
                    (_FakeTensor(8), _lib.DTYPE_F16),
                    (None, _lib.DTYPE_F32)):
        with pytest.raises(ValueError):
            _dev_tensor(t, 8, code, "x")


def test_projection_tensors_are_checked_on_the_host():
    from qauntrunner_amd.weights import _f32_dev, _weight_dev

    assert _f32_dev(_FakeTensor(12), "x", multiple=4) == 3
    assert _f32_dev(_FakeTensor(12), "y", numel=12) == 0
    assert _f32_dev(_FakeTensor(16), "y", numel=12) == 0               # a larger output buffer
    for t, kw in ((_FakeTensor(13), {"multiple": 4}),                  # not whole rows
                  (_FakeTensor(11), {"numel": 12}),                    # short output
                  (_FakeTensor(12, cuda=False), {"numel": 12}),        # host tensor
                  (_FakeTensor(12, contiguous=False), {"numel": 12}),  # strided view
                  (_FakeTensor(12, "torch.float16"), {"numel": 12})):  # wrong element type
        with pytest.raises(ValueError):
            _f32_dev(t, "x", **kw)

    class _Raw(_FakeTensor):
        def element_size(self):
            return 1
    _weight_dev(_Raw(64 * 1024 * 2, "torch.uint8"), "F16", 64, 1024, "w")  # 64 rows of 2 KiB: enough
    with pytest.raises(ValueError):
        _weight_dev(_Raw(64 * 1024 * 2 - 1, "torch.uint8"), "F16", 64, 1024, "w")
    with pytest.raises(ValueError):
        _weight_dev(_Raw(64 * 1024 * 2, "torch.uint8", cuda=False), "F16", 64, 1024, "w")


def test_device_position_tensors_are_checked_on_the_host():
    from qauntrunner_amd.caches import _dev_int32

    assert _dev_int32(_FakeTensor(1, "torch.int32"), 1, "pos").value == 0x1000
    for t in (_FakeTensor(2, "torch.int32"), _FakeTensor(1, "torch.int64"), _FakeTensor(1, "torch.int32", cuda=False),
              _FakeTensor(1, "torch.int32", contiguous=False), None):
        with pytest.raises(ValueError):
            _dev_int32(t, 1, "pos")


def test_projection_weights_are_checked_against_the_call():
    """A store DeviceTensor handed to a *_dev projection must match the call's format and hold
    the rows it reads; the check runs on the host, before any device address is used."""
    from qauntrunner_amd.store import DeviceTensor, TensorView
    from qauntrunner_amd.weights import _weight_dev, row_bytes

    dt = DeviceTensor(TensorView("l0.wq", (8, 256), 4, 8 * row_bytes(4, 256)), 0x1000)  # Q8_0 [8 x 256]
    _weight_dev(dt, 4, 8, 256, "w")
    with pytest.raises(ValueError, match="format"):
        _weight_dev(dt, 6, 8, 256, "w")
    with pytest.raises(ValueError, match="bytes"):
        _weight_dev(dt, 4, 16, 256, "w")
    with pytest.raises(ValueError, match="expected a Weight"):
        _weight_dev(object(), 4, 8, 256, "w")
