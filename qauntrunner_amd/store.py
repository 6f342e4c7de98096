""".qw weight files served from HBM: ModelStore and PrefetchPipeline.

``ModelStore`` mirrors Core/Memory/ModelStore.cs (Open, Tensors, Get, Has) over
the ``qr_model`` handle of libqr_attn; ``PrefetchPipeline`` mirrors
Core/Runtime/PrefetchPipeline.cs (Begin, Acquire, WaitLayer and the counters)
with HBM ping-pong slots in place of the pinned host buffers, so Acquire
returns a device address.  ``ModelStoreBuilder`` writes the same file layout as
ModelStoreBuilder.Commit (ModelStore.cs:143-229).
"""
from __future__ import annotations

import ctypes
import json
import struct

import numpy as np

from . import _lib
from ._lib import check

__all__ = ["ModelStore", "PrefetchPipeline", "ModelStoreBuilder", "TensorView", "DeviceTensor"]

MAGIC = b"QWR1"


class TensorView:
    """Name, Dims, Format and SizeBytes of one tensor (ModelStore.cs:10-43)."""

    def __init__(self, name, dims, fmt, size):
        self.Name, self.Dims, self.Format, self.SizeBytes = name, tuple(dims), fmt, size

    @property
    def NumElements(self) -> int:
        n = 1
        for d in self.Dims:
            n *= d
        return n

    def RowBytes(self) -> int:
        """TensorView.RowBytes (ModelStore.cs:37-42): bytes of one row of Dims[-1] values."""
        from .weights import row_bytes

        return row_bytes(self.Format, self.Dims[-1])

    def __repr__(self):
        return f"TensorView({self.Name!r}, dims={self.Dims}, format={self.Format}, bytes={self.SizeBytes})"


class DeviceTensor:
    """A device address handed out by Acquire; ``data_ptr()`` lets the projections take it."""

    def __init__(self, view: TensorView, ptr: int):
        self.View, self._ptr = view, ptr

    def data_ptr(self) -> int:
        return self._ptr


class ModelStore:
    """ModelStore.Open (ModelStore.cs:85-126) on a .qw file; the file stays open."""

    def __init__(self, path: str):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.qr_model_open(ctypes.byref(h), path.encode()))
        self._h = h
        _lib.track(self)
        self.Path = path
        n = ctypes.c_int()
        check(self._lib.qr_model_tensor_count(h, ctypes.byref(n)))
        self.Tensors = {}
        buf = ctypes.create_string_buffer(4096)
        for i in range(n.value):
            check(self._lib.qr_model_tensor_name(h, i, buf, len(buf)))
            name = buf.value.decode()
            self.Tensors[name] = self._info(name)

    @staticmethod
    def Open(path: str) -> "ModelStore":
        return ModelStore(path)

    def _info(self, name: str) -> TensorView:
        fmt, nd, size = ctypes.c_int(), ctypes.c_int(), ctypes.c_longlong()
        dims = (ctypes.c_longlong * 16)()
        check(self._lib.qr_model_tensor_info(self._h, name.encode(), ctypes.byref(fmt), ctypes.byref(nd), dims, 16,
                                             ctypes.byref(size)))
        return TensorView(name, [dims[i] for i in range(nd.value)], fmt.value, size.value)

    @property
    def handle(self):
        return self._h

    def Has(self, name: str) -> bool:
        return name in self.Tensors

    def Get(self, name: str) -> TensorView:
        if name not in self.Tensors:
            raise KeyError(f"tensor '{name}' not found in {self.Path}")
        return self.Tensors[name]

    def Read(self, name: str) -> np.ndarray:
        """TensorView.Bytes (ModelStore.cs:27) as a host uint8 array."""
        v = self.Get(name)
        out = np.empty(v.SizeBytes, np.uint8)
        check(self._lib.qr_model_read(self._h, name.encode(), out.ctypes.data_as(ctypes.c_void_p), out.size))
        return out

    def MakeResident(self) -> None:
        """Every tensor uploaded once to the current device; Acquire then never copies or waits."""
        check(self._lib.qr_model_make_resident(self._h))

    def Dispose(self) -> None:
        if getattr(self, "_h", None):
            check(self._lib.qr_model_close(self._h))
            self._h = None

    close = Dispose

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.Dispose()

    def __del__(self):
        if _lib.finalizing():  # the exit hook closed what was open; the runtime may be gone
            return
        try:
            self.Dispose()
        except Exception:
            pass


def _stream(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(getattr(stream, "cuda_stream", stream))


class PrefetchPipeline:
    """PrefetchPipeline (PrefetchPipeline.cs:19-190) staging layers into two HBM slots."""

    def __init__(self, store: ModelStore, budget_bytes: int):
        self._store, self._lib = store, store._lib
        self._budget = int(budget_bytes)
        check(self._lib.qr_model_set_prefetch(store.handle, self._budget))

    @property
    def Enabled(self) -> bool:
        return self._budget > 0

    def Begin(self, layer: int) -> None:
        check(self._lib.qr_model_begin(self._store.handle, layer))

    def Acquire(self, name: str, layer: int, stream=None) -> DeviceTensor:
        p = ctypes.c_void_p()
        check(self._lib.qr_model_acquire(self._store.handle, name.encode(), layer, _stream(stream), ctypes.byref(p)))
        return DeviceTensor(self._store.Get(name), p.value)

    def Release(self, layer: int, stream=None) -> None:
        check(self._lib.qr_model_release(self._store.handle, layer, _stream(stream)))

    def WaitLayer(self, layer: int) -> None:
        check(self._lib.qr_model_wait_layer(self._store.handle, layer))

    def _stats(self):
        b, w, r = ctypes.c_longlong(), ctypes.c_double(), ctypes.c_double()
        s, k = ctypes.c_int(), ctypes.c_int()
        check(self._lib.qr_model_stats(self._store.handle, ctypes.byref(b), ctypes.byref(w), ctypes.byref(r),
                                       ctypes.byref(s), ctypes.byref(k)))
        return b.value, w.value, r.value, s.value, k.value

    @property
    def BytesStreamed(self) -> int:
        return self._stats()[0]

    @property
    def WaitMs(self) -> float:
        return self._stats()[1]

    @property
    def ReadMs(self) -> float:
        return self._stats()[2]

    @property
    def StagedLayers(self) -> int:
        return self._stats()[3]

    @property
    def SkippedLayers(self) -> int:
        return self._stats()[4]

    def Dispose(self) -> None:
        if self._store.handle:
            check(self._lib.qr_model_set_prefetch(self._store.handle, 0))
            self._budget = 0


class ModelStoreBuilder:
    """Writes a .qw file in ModelStoreBuilder.Commit's layout (ModelStore.cs:173-229):
    "QWR1", int32 header length, the JSON header, zero padding to the 64-byte-aligned data
    start, then the tensors back to back in plan order.  header_reserve_bytes > 0 records an
    absolute data_offset (ModelStore.cs:201-209)."""

    def __init__(self, path: str, config: dict, header_reserve_bytes: int = 0):
        self.path, self.config = path, config
        self.reserve = max(0, int(header_reserve_bytes))
        self.plans = []

    def Plan(self, name: str, dims, fmt, size_bytes: int) -> None:
        self.plans.append((name, [int(d) for d in dims], int(fmt), int(size_bytes)))

    def Commit(self, write_tensor) -> None:
        """write_tensor(name) returns the tensor's bytes (exactly the planned size)."""
        entries, off = [], 0
        for name, dims, fmt, size in self.plans:
            entries.append({"name": name, "dims": dims, "format": fmt, "offset": off, "size": size})
            off += size
        header = {"config": self.config, "tensors": entries}
        hb = json.dumps(header, separators=(",", ":")).encode()
        if self.reserve:
            data_start = (8 + self.reserve + 63) & ~63
            header["data_offset"] = data_start
            hb = json.dumps(header, separators=(",", ":")).encode()
            if 8 + len(hb) > data_start:
                raise IOError(f"header needs {len(hb)} bytes, reserved region only {self.reserve}")
        else:
            data_start = (8 + len(hb) + 63) & ~63
        with open(self.path, "wb") as f:
            f.write(MAGIC + struct.pack("<i", len(hb)) + hb)
            f.write(b"\0" * (data_start - 8 - len(hb)))
            for name, _, _, size in self.plans:
                data = np.ascontiguousarray(write_tensor(name), dtype=np.uint8).reshape(-1)
                if data.size != size:
                    raise IOError(f"tensor '{name}': wrote {data.size} bytes, planned {size}")
                f.write(data.tobytes())
