"""HBM-resident weight tensors and the MLA projections over them.

``Weight`` is one tensor of a ModelStore (ModelStore.cs: a format, a row count,
``RowBytes`` per row) uploaded once to the GPU; the projections decode its rows
on the fly exactly as BlockDequantizer.Dequantize (Core/Quantization/
BlockDequantizer.cs) and follow the reference's fp32 operation order, so their
results equal the reference's bit for bit.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import FORMATS, check

__all__ = ["Weight", "row_bytes", "format_code", "mla_q_absorb_dev", "mla_wuv_dev", "matvec_dev", "matvec_group_dev"]


def format_code(fmt) -> int:
    return fmt if isinstance(fmt, int) else FORMATS[fmt]


def row_bytes(fmt, cols: int) -> int:
    """Bytes of one row of `cols` weights (Dtypes.TensorBytes)."""
    out = ctypes.c_longlong()
    check(_lib.load().qr_weight_row_bytes(format_code(fmt), cols, ctypes.byref(out)))
    return out.value


class Weight:
    """A [rows, cols] weight tensor in one QuantFormat, uploaded from its raw bytes."""

    def __init__(self, fmt, rows: int, cols: int, raw: np.ndarray):
        self._lib = _lib.load()
        self.Fmt = format_code(fmt)
        self.Rows, self.Cols = rows, cols
        self.RowBytes = row_bytes(self.Fmt, cols)
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        if raw.size != rows * self.RowBytes:
            raise ValueError(f"expected {rows * self.RowBytes} bytes, got {raw.size}")
        h = ctypes.c_void_p()
        check(self._lib.qr_weight_create(ctypes.byref(h), self.Fmt, rows, cols,
                                          raw.ctypes.data_as(ctypes.c_void_p)))
        self._h = h
        _lib.track(self)

    @property
    def handle(self):
        return self._h

    def data_ptr(self) -> int:
        p = ctypes.c_void_p()
        check(self._lib.qr_weight_data(self._h, ctypes.byref(p)))
        return p.value

    def MatVec(self, x) -> np.ndarray:
        """DotKernels.MatVec: y = W x for host x [cols] or [nq][cols]; returns [nq][rows] (or [rows])."""
        xa = np.ascontiguousarray(x, dtype=np.float32)
        nq = xa.size // self.Cols
        if xa.size != nq * self.Cols:
            raise ValueError(f"x must hold a multiple of {self.Cols} values")
        y = np.empty((nq, self.Rows), np.float32)
        check(self._lib.qr_matvec(self._h, nq, xa.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p)))
        return y if xa.ndim > 1 else y[0]

    def close(self):
        if getattr(self, "_h", None):
            self._lib.qr_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        if _lib.finalizing():  # the exit hook closed what was open; the runtime may be gone
            return
        try:
            self.close()
        except Exception:
            pass


def _dev(x):
    """Device address of a Weight or of a torch tensor."""
    return ctypes.c_void_p(x.data_ptr())


def _stream(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(getattr(stream, "cuda_stream", stream))


def _f32_dev(t, what, numel=None, multiple=None) -> int:
    """Checks an fp32 torch tensor handed to a *_dev projection before its address reaches a
    kernel (the C ABI cannot see device sizes): on the GPU, contiguous, float32, and either
    at least `numel` elements (an output: the call writes the first `numel`) or a whole
    number of `multiple`-element rows (an input whose rows set the vector count).  Returns
    the rows."""
    if not getattr(t, "is_cuda", False):
        raise ValueError(f"{what}: expected a tensor on the GPU")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    if str(t.dtype) != "torch.float32":
        raise ValueError(f"{what}: expected float32, got {t.dtype}")
    if numel is not None and t.numel() < numel:
        raise ValueError(f"{what}: {t.numel()} elements, the call writes {numel}")
    if multiple is not None and (multiple <= 0 or t.numel() % multiple):
        raise ValueError(f"{what}: {t.numel()} elements are not whole rows of {multiple}")
    return t.numel() // multiple if multiple else 0


def _weight_dev(w, fmt, rows, cols, what) -> None:
    """A weight handed to a *_dev call must hold `rows` rows of `cols` weights in format
    `fmt` before its address reaches a kernel: a Weight is checked against its own format
    and shape, a store DeviceTensor against its view's format and byte size, a raw torch
    tensor (a contiguous GPU buffer) against its byte size."""
    code = format_code(fmt)
    need = rows * row_bytes(code, cols)
    if isinstance(w, Weight):
        if (w.Fmt, w.Rows, w.Cols) != (code, rows, cols):
            raise ValueError(f"{what}: the Weight is format {w.Fmt} [{w.Rows} x {w.Cols}], "
                             f"the call reads format {code} [{rows} x {cols}]")
        return
    view = getattr(w, "View", None)
    if view is not None:  # a store DeviceTensor
        if view.Format != code:
            raise ValueError(f"{what}: tensor {view.Name} is format {view.Format}, the call reads format {code}")
        if view.SizeBytes < need:
            raise ValueError(f"{what}: tensor {view.Name} holds {view.SizeBytes} bytes, {need} needed")
        return
    if hasattr(w, "is_cuda"):
        if not w.is_cuda or not w.is_contiguous():
            raise ValueError(f"{what}: expected a contiguous tensor on the GPU")
        if w.numel() * w.element_size() < need:
            raise ValueError(f"{what}: {w.numel() * w.element_size()} bytes, {need} needed")
        return
    raise ValueError(f"{what}: expected a Weight, a store DeviceTensor or a torch tensor on the GPU")


def mla_q_absorb_dev(kvb, fmt, heads, nope, rope, vdim, kv_lora, q, q_tilde, stream=None) -> None:
    """q_tilde[b,h,:] = sum_j q[b,h,j] * W_kvb[h*(nope+vdim)+j, :] (StreamingEngine.cs:517-529)."""
    _weight_dev(kvb, fmt, heads * (nope + vdim), kv_lora, "kvb")
    nq = _f32_dev(q, "q", multiple=heads * (nope + rope))
    _f32_dev(q_tilde, "q_tilde", numel=nq * heads * kv_lora)
    check(_lib.load().qr_mla_q_absorb_dev(_dev(kvb), format_code(fmt), heads, nope, rope, vdim, kv_lora, nq,
                                          ctypes.c_void_p(q.data_ptr()), ctypes.c_void_p(q_tilde.data_ptr()),
                                          _stream(stream)))


def mla_wuv_dev(kvb, fmt, heads, nope, vdim, kv_lora, u, out, stream=None) -> None:
    """out[b,h,j] = DotF32(W_kvb[h*(nope+vdim)+nope+j, :], u[b,h]) (StreamingEngine.cs:569-576)."""
    _weight_dev(kvb, fmt, heads * (nope + vdim), kv_lora, "kvb")
    nq = _f32_dev(u, "u", multiple=heads * kv_lora)
    _f32_dev(out, "out", numel=nq * heads * vdim)
    check(_lib.load().qr_mla_wuv_dev(_dev(kvb), format_code(fmt), heads, nope, vdim, kv_lora, nq,
                                     ctypes.c_void_p(u.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                     _stream(stream)))


def matvec_group_dev(ws, fmt, rows, cols, x, ys, stream=None) -> None:
    """MatVecs of up to 4 weights against the same x in one launch where the format allows
    (qr_matvec_group_dev): ys[m][b, r] = DotRow(ws[m] row r, x[b])."""
    n = len(ws)
    if not (len(rows) == n == len(ys)):
        raise ValueError("ws, rows and ys must have the same length")
    nq = _f32_dev(x, "x", multiple=cols)
    for m in range(n):
        _weight_dev(ws[m], fmt, rows[m], cols, f"ws[{m}]")
        _f32_dev(ys[m], f"ys[{m}]", numel=nq * rows[m])
    wp = (ctypes.c_void_p * n)(*[w.data_ptr() for w in ws])
    rp = (ctypes.c_longlong * n)(*rows)
    yp = (ctypes.c_void_p * n)(*[y.data_ptr() for y in ys])
    check(_lib.load().qr_matvec_group_dev(n, wp, rp, format_code(fmt), cols, nq, ctypes.c_void_p(x.data_ptr()), yp,
                                          _stream(stream)))


def matvec_dev(w, fmt, rows, cols, x, y, stream=None) -> None:
    """y[b, r] = DotRow(W row r, x[b]) on device tensors (DotKernels.cs:599-633)."""
    _weight_dev(w, fmt, rows, cols, "w")
    nq = _f32_dev(x, "x", multiple=cols)
    _f32_dev(y, "y", numel=nq * rows)
    check(_lib.load().qr_matvec_dev(_dev(w), format_code(fmt), rows, cols, nq, ctypes.c_void_p(x.data_ptr()),
                                    ctypes.c_void_p(y.data_ptr()), _stream(stream)))
