"""Host-side mirror of QuantRunner's attention caches over libqr_attn.

``PagedKvCache`` and ``MlaLatentCache`` keep the member names and argument
meaning of the C# classes (src/QuantRunner.Core/Runtime/PagedKvCache.cs,
MlaLatentCache.cs) and forward every call to the C ABI.  Host-array calls
take numpy arrays (fp32, or uint16 bit patterns for 16-bit data) and are
synchronous; the ``*Dev`` calls take torch tensors already on the GPU and
enqueue on torch's current stream.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import DTYPES, PAGE_TOKENS, check

__all__ = ["PagedKvCache", "MlaLatentCache", "dtype_code"]


def dtype_code(dt) -> int:
    if isinstance(dt, int):
        return dt
    return DTYPES[dt]


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _host_rows(x, src_dtype: int):
    """Contiguous host rows: fp32 for DTYPE_F32, uint16 bit patterns otherwise."""
    want = np.float32 if src_dtype == _lib.DTYPE_F32 else np.uint16
    a = np.ascontiguousarray(x)
    if a.dtype != want:
        raise TypeError(f"expected {np.dtype(want).name} rows for dtype code {src_dtype}, got {a.dtype}")
    return a


def _dev_ptr(x):
    """Device address of a torch tensor or of a weights.Weight."""
    return ctypes.c_void_p(x.data_ptr())


_TORCH_CODES = {"float32": 0, "float16": 1, "bfloat16": 2, "int16": -1, "uint16": -1}


def _dev_tensor(x, numel, code, what, allow_none=False):
    """Checks a torch tensor handed to a *Dev call before its address reaches a kernel:
    on the GPU, contiguous, `numel` elements of the element type of dtype `code`
    (fp32 for DTYPE_F32; 2-byte elements -- fp16, bf16 or int16/uint16 bit patterns --
    for the 16-bit codes).  The C ABI cannot see device sizes, so a short tensor would
    otherwise be read or written out of bounds."""
    if x is None:
        if allow_none:
            return ctypes.c_void_p()
        raise ValueError(f"{what}: tensor required")
    if not getattr(x, "is_cuda", False):
        raise ValueError(f"{what}: expected a tensor on the GPU")
    if not x.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")
    name = str(x.dtype).replace("torch.", "")
    tc = _TORCH_CODES.get(name)
    ok = tc == code if code == _lib.DTYPE_F32 else tc is not None and tc != _lib.DTYPE_F32 and (tc in (-1, code))
    if not ok:
        raise ValueError(f"{what}: dtype {name} does not match dtype code {code}")
    if x.numel() != numel:
        raise ValueError(f"{what}: expected {numel} elements, got {x.numel()}")
    return ctypes.c_void_p(x.data_ptr())


def _dev_int32(x, numel, what):
    """Checks a device int32 tensor (positions read by the kernels) the same way."""
    if x is None or not getattr(x, "is_cuda", False):
        raise ValueError(f"{what}: expected an int32 tensor on the GPU")
    if not x.is_contiguous() or str(x.dtype) != "torch.int32":
        raise ValueError(f"{what}: expected a contiguous int32 tensor")
    if x.numel() != numel:
        raise ValueError(f"{what}: expected {numel} elements, got {x.numel()}")
    return ctypes.c_void_p(x.data_ptr())


def _rows_of(x, width, what):
    n = x.numel() // width if x is not None else 0
    if x is None or n * width != x.numel():
        raise ValueError(f"{what}: element count must be a multiple of {width}")
    return n


def _stream_ptr(stream):
    if stream is None:
        import torch

        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return ctypes.c_void_p(getattr(stream, "cuda_stream", stream))


class PagedKvCache:
    """Paged K/V store with fused GQA decode attention (PagedKvCache.cs:12-136)."""

    PageTokens = PAGE_TOKENS  # PagedKvCache.cs:14

    def __init__(self, layers, heads, kv_heads, head_dim, max_seq, kv_dtype="f32", max_batch=1):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        check(self._lib.qr_kv_create(ctypes.byref(h), layers, heads, kv_heads, head_dim, max_seq,
                                     dtype_code(kv_dtype), max_batch))
        self._h = h
        _lib.track(self)
        self.Layers, self.Heads, self.KvHeads, self.HeadDim = layers, heads, kv_heads, head_dim
        self.MaxSeq, self.MaxBatch = max_seq, max_batch
        self.KvDtype = dtype_code(kv_dtype)
        self.KvDim = kv_heads * head_dim

    # ---- lifetime
    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            check(self._lib.qr_kv_destroy(self._h))
            self._h = None

    def __del__(self):
        if _lib.finalizing():  # the exit hook closed what was open; the runtime may be gone
            return
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- properties
    def seq_len(self, seq_id=0) -> int:
        out = ctypes.c_int()
        check(self._lib.qr_kv_seq_len(self._h, seq_id, ctypes.byref(out)))
        return out.value

    @property
    def SeqLen(self) -> int:  # PagedKvCache.cs:26
        return self.seq_len(0)

    @property
    def BytesUsed(self) -> int:  # PagedKvCache.cs:27
        out = ctypes.c_longlong()
        check(self._lib.qr_kv_bytes_used(self._h, ctypes.byref(out)))
        return out.value

    @property
    def BytesPerToken(self) -> int:  # PagedKvCache.cs:39
        out = ctypes.c_longlong()
        check(self._lib.qr_kv_bytes_per_token(self._h, ctypes.byref(out)))
        return out.value

    def Reserve(self, pages: int) -> None:
        check(self._lib.qr_kv_reserve(self._h, pages))

    def SetSplitEvent(self, event) -> None:
        """Benchmark instrumentation: record hipEvent_t `event` after every split-K kernel (None: off)."""
        check(self._lib.qr_kv_set_split_event(self._h, event))

    # ---- writes
    def Append(self, layer, pos, k, v, seq_id=0) -> None:
        """PagedKvCache.Append (:62-69): fp32 rows of at most kv_dim floats."""
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        check(self._lib.qr_kv_append(self._h, seq_id, layer, pos, _ptr(k), k.size, _ptr(v), v.size))

    def AppendRange(self, layer, pos0, k_rows, v_rows, src_dtype="f32", seq_id=0) -> None:
        code = dtype_code(src_dtype)
        k = _host_rows(k_rows, code)
        v = _host_rows(v_rows, code)
        n = k.size // self.KvDim
        if k.size != n * self.KvDim or v.size != k.size:
            raise ValueError("k/v rows must both be [n, kv_dim]")
        check(self._lib.qr_kv_append_range(self._h, seq_id, layer, pos0, n, _ptr(k), _ptr(v), code))

    def AppendRangeDev(self, layer, pos0, k_rows, v_rows, src_dtype="f32", seq_id=0, stream=None) -> None:
        code = dtype_code(src_dtype)
        n = _rows_of(k_rows, self.KvDim, "k rows")
        kp = _dev_tensor(k_rows, n * self.KvDim, code, "k rows")
        vp = _dev_tensor(v_rows, n * self.KvDim, code, "v rows")
        check(self._lib.qr_kv_append_range_dev(self._h, seq_id, layer, pos0, n, kp, vp, code, _stream_ptr(stream)))

    def AppendRope(self, layer, pos, q, k, v, theta, seq_id=0) -> np.ndarray:
        """StreamingEngine.cs:245-248: RoPE on q and k at `pos` (TransformerOps.cs:56-88),
        then Append(k, v).  Returns the rotated q (the reference rotates it in place)."""
        q = np.array(q, dtype=np.float32, copy=True).reshape(-1)
        k = np.ascontiguousarray(k, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(v, dtype=np.float32).reshape(-1)
        if q.size != self.Heads * self.HeadDim or k.size != self.KvDim or v.size != self.KvDim:
            raise ValueError("q must be heads*head_dim floats, k and v kv_dim floats")
        check(self._lib.qr_kv_append_rope(self._h, seq_id, layer, pos, _ptr(q), _ptr(k), _ptr(v), theta))
        return q

    def AppendRopeDev(self, layer, pos0, q_rows, k_rows, v_rows, theta, seq_id=0, stream=None) -> None:
        """n positions from device rows; q_rows (or None) is rotated in place."""
        f32 = _lib.DTYPE_F32
        n = _rows_of(k_rows, self.KvDim, "k rows")
        qp = _dev_tensor(q_rows, n * self.Heads * self.HeadDim, f32, "q rows", allow_none=True)
        kp = _dev_tensor(k_rows, n * self.KvDim, f32, "k rows")
        vp = _dev_tensor(v_rows, n * self.KvDim, f32, "v rows")
        check(self._lib.qr_kv_append_rope_dev(self._h, seq_id, layer, pos0, n, qp, kp, vp, theta,
                                              _stream_ptr(stream)))

    def AppendRopeStepDev(self, layer, pos_dev, q_row, k_row, v_row, theta, seq_id=0, stream=None) -> None:
        """AppendRopeDev of one position whose index is read on the GPU from pos_dev (int32
        [1]); its page is claimed on the device, so the call can be captured in a graph and
        replayed at advancing positions (pages must be reserved before capture)."""
        f32 = _lib.DTYPE_F32
        pp = _dev_int32(pos_dev, 1, "pos")
        qp = _dev_tensor(q_row, self.Heads * self.HeadDim, f32, "q row", allow_none=True)
        kp = _dev_tensor(k_row, self.KvDim, f32, "k row")
        vp = _dev_tensor(v_row, self.KvDim, f32, "v row")
        check(self._lib.qr_kv_append_rope_step_dev(self._h, seq_id, layer, pp, qp, kp, vp, theta,
                                                   _stream_ptr(stream)))

    def AppendRopeChunkStepDev(self, layer, pos0_dev, q_rows, k_rows, v_rows, theta, seq_id=0,
                               stream=None) -> None:
        """AppendRopeStepDev of nq consecutive positions from pos0_dev (int32 [1]) on: q
        [nq, heads*head_dim] (rotated in place, or None), k/v [nq, kv_heads*head_dim]."""
        f32 = _lib.DTYPE_F32
        nq = _rows_of(k_rows, self.KvDim, "k rows")
        pp = _dev_int32(pos0_dev, 1, "pos0")
        qp = _dev_tensor(q_rows, nq * self.Heads * self.HeadDim, f32, "q rows", allow_none=True)
        kp = _dev_tensor(k_rows, nq * self.KvDim, f32, "k rows")
        vp = _dev_tensor(v_rows, nq * self.KvDim, f32, "v rows")
        check(self._lib.qr_kv_append_rope_chunk_step_dev(self._h, seq_id, layer, nq, pp, qp, kp, vp, theta,
                                                         _stream_ptr(stream)))

    def Reset(self, seq_id=-1) -> None:  # PagedKvCache.cs:72
        check(self._lib.qr_kv_reset(self._h, seq_id))

    def Truncate(self, length, seq_id=0) -> None:  # PagedKvCache.cs:76
        check(self._lib.qr_kv_truncate(self._h, seq_id, length))

    # ---- attention
    def Attention(self, layer, pos, q, scale, seq_id=0) -> np.ndarray:
        """PagedKvCache.Attention (:83-136); returns attn [heads*head_dim] fp32."""
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        if q.size != self.Heads * self.HeadDim:
            raise ValueError(f"q must hold heads*head_dim = {self.Heads * self.HeadDim} floats")
        out = np.empty(self.Heads * self.HeadDim, np.float32)
        check(self._lib.qr_kv_attention(self._h, seq_id, layer, pos, _ptr(q), _ptr(out), scale))
        return out

    def AttentionBatch(self, layer, seq_ids, positions, q, scale) -> np.ndarray:
        ids = np.ascontiguousarray(seq_ids, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        n = ids.size
        q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
        if pos.size != n or q.size != n * self.Heads * self.HeadDim:
            raise ValueError("seq_ids, positions and q rows must agree")
        out = np.empty((n, self.Heads * self.HeadDim), np.float32)
        check(self._lib.qr_kv_attention_batch(self._h, n, _ptr(ids), layer, _ptr(pos), _ptr(q), _ptr(out), scale))
        return out

    def AttentionDev(self, layer, seq_ids, positions, q, out, scale, stream=None) -> None:
        ids = np.ascontiguousarray(seq_ids, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        if pos.size != ids.size:
            raise ValueError("seq_ids and positions must agree")
        rows = ids.size * self.Heads * self.HeadDim
        qp = _dev_tensor(q, rows, _lib.DTYPE_F32, "q")
        op = _dev_tensor(out, rows, _lib.DTYPE_F32, "out")
        check(self._lib.qr_kv_attention_dev(self._h, ids.size, _ptr(ids), layer, _ptr(pos), qp, op, scale,
                                            _stream_ptr(stream)))

    def AttentionDevNoAlloc(self, layer, seq_ids, positions, q, out, scale, stream=None) -> None:
        """AttentionDev through qr_kv_attention_dev_noalloc: split partials in the library's
        fixed device array, no allocation (at most 64 entries, 8 MiB - 64 KiB of partials)."""
        ids = np.ascontiguousarray(seq_ids, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        if pos.size != ids.size:
            raise ValueError("seq_ids and positions must agree")
        rows = ids.size * self.Heads * self.HeadDim
        qp = _dev_tensor(q, rows, _lib.DTYPE_F32, "q")
        op = _dev_tensor(out, rows, _lib.DTYPE_F32, "out")
        check(self._lib.qr_kv_attention_dev_noalloc(self._h, ids.size, _ptr(ids), layer, _ptr(pos), qp, op, scale,
                                                    _stream_ptr(stream)))

    def AttentionStepDev(self, layer, seq_ids, pos_dev, q, out, scale, stream=None) -> None:
        """AttentionDev with the positions read on the GPU from pos_dev (int32, one per entry):
        entry i attends positions 0..pos_dev[i] (graph-capturable; the split count is planned
        for max_seq and each entry spreads over it on the device)."""
        ids = np.ascontiguousarray(seq_ids, dtype=np.int32)
        rows = ids.size * self.Heads * self.HeadDim
        pp = _dev_int32(pos_dev, ids.size, "pos")
        qp = _dev_tensor(q, rows, _lib.DTYPE_F32, "q")
        op = _dev_tensor(out, rows, _lib.DTYPE_F32, "out")
        check(self._lib.qr_kv_attention_step_dev(self._h, ids.size, _ptr(ids), layer, pp, qp, op, scale,
                                                 _stream_ptr(stream)))

    def DecodePlan(self, layer, seq_ids, positions):
        """(tokens per split, splits of the longest entry) that a decode call with these
        entries takes."""
        ids = np.ascontiguousarray(seq_ids, dtype=np.int32)
        pos = np.ascontiguousarray(positions, dtype=np.int32)
        if pos.size != ids.size:
            raise ValueError("seq_ids and positions must agree")
        st, ns = ctypes.c_int(), ctypes.c_int()
        check(self._lib.qr_kv_decode_plan(self._h, ids.size, _ptr(ids), layer, _ptr(pos), ctypes.byref(st),
                                          ctypes.byref(ns)))
        return st.value, ns.value

    def AttentionChunk(self, layer, pos0, q, scale, q_dtype="f32", seq_id=0) -> np.ndarray:
        """Causal attention of nq queries at pos0..pos0+nq-1 (each sees 0..its position)."""
        code = dtype_code(q_dtype)
        q = _host_rows(q, code)
        row = self.Heads * self.HeadDim
        nq = q.size // row
        if q.size != nq * row:
            raise ValueError("q must be [nq, heads*head_dim]")
        out = np.empty((nq, row), np.float32)
        check(self._lib.qr_kv_attention_chunk(self._h, seq_id, layer, pos0, nq, _ptr(q), code, _ptr(out), scale))
        return out

    def AttentionChunkDev(self, layer, pos0, q, out, scale, q_dtype="f32", seq_id=0, stream=None) -> None:
        row = self.Heads * self.HeadDim
        code = dtype_code(q_dtype)
        nq = _rows_of(q, row, "q")
        qp = _dev_tensor(q, nq * row, code, "q")
        op = _dev_tensor(out, nq * row, _lib.DTYPE_F32, "out")
        check(self._lib.qr_kv_attention_chunk_dev(self._h, seq_id, layer, pos0, nq, qp, code, op, scale,
                                                  _stream_ptr(stream)))

    def AttentionChunkStepDev(self, layer, pos0_dev, q, out, scale, q_dtype="f32", seq_id=0, stream=None) -> None:
        """AttentionChunkDev with the position of query 0 read on the GPU from pos0_dev (int32
        [1]); graph-capturable like AttentionStepDev."""
        row = self.Heads * self.HeadDim
        code = dtype_code(q_dtype)
        nq = _rows_of(q, row, "q")
        pp = _dev_int32(pos0_dev, 1, "pos0")
        qp = _dev_tensor(q, nq * row, code, "q")
        op = _dev_tensor(out, nq * row, _lib.DTYPE_F32, "out")
        check(self._lib.qr_kv_attention_chunk_step_dev(self._h, seq_id, layer, nq, pp, qp, code, op, scale,
                                                       _stream_ptr(stream)))

    # ---- debug copy-out
    def Read(self, layer, pos0, n, seq_id=0):
        """Rows pos0..pos0+n-1 as stored (fp32, or uint16 bits for 16-bit caches)."""
        dt = np.float32 if self.KvDtype == _lib.DTYPE_F32 else np.uint16
        k = np.empty((n, self.KvDim), dt)
        v = np.empty((n, self.KvDim), dt)
        check(self._lib.qr_kv_read(self._h, seq_id, layer, pos0, n, _ptr(k), _ptr(v)))
        return k, v


class MlaLatentCache:
    """Paged MLA latent store with absorbed attention (MlaLatentCache.cs:10-65,
    StreamingEngine.cs:531-568).

    MlaLatentCache(layers, latentDim, maxSeq) as the reference's constructor takes it;
    `rope` (the k_pe width at the end of each latent row) splits the row for attention
    and may instead be set later with SetRope, as MlaLayer knows it."""

    PageTokens = PAGE_TOKENS

    def __init__(self, layers, latent_dim, max_seq, dtype="f32", rope=None):
        self._lib = _lib.load()
        h = ctypes.c_void_p()
        if rope is None:
            check(self._lib.qr_mla_create_latent(ctypes.byref(h), layers, latent_dim, max_seq, dtype_code(dtype)))
        else:
            check(self._lib.qr_mla_create(ctypes.byref(h), layers, latent_dim - rope, rope, max_seq,
                                          dtype_code(dtype)))
        self._h = h
        _lib.track(self)
        self.Layers, self.MaxSeq = layers, max_seq
        self.LatentDim = latent_dim
        self.Rope = rope
        self.KvLora = latent_dim - rope if rope is not None else None
        self.Dtype = dtype_code(dtype)

    def SetRope(self, rope) -> None:
        check(self._lib.qr_mla_set_rope(self._h, rope))
        self.Rope, self.KvLora = rope, self.LatentDim - rope

    def max_seq(self) -> int:
        out = ctypes.c_int()
        check(self._lib.qr_mla_max_seq(self._h, ctypes.byref(out)))
        return out.value

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            check(self._lib.qr_mla_destroy(self._h))
            self._h = None

    def __del__(self):
        if _lib.finalizing():  # the exit hook closed what was open; the runtime may be gone
            return
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def SeqLen(self) -> int:
        out = ctypes.c_int()
        check(self._lib.qr_mla_seq_len(self._h, ctypes.byref(out)))
        return out.value

    @property
    def BytesUsed(self) -> int:
        out = ctypes.c_longlong()
        check(self._lib.qr_mla_bytes_used(self._h, ctypes.byref(out)))
        return out.value

    def PageCount(self, layer) -> int:
        out = ctypes.c_int()
        check(self._lib.qr_mla_page_count(self._h, layer, ctypes.byref(out)))
        return out.value

    def Page(self, layer, page) -> np.ndarray:
        out = np.empty((PAGE_TOKENS, self.LatentDim), np.float32)
        check(self._lib.qr_mla_read_page(self._h, layer, page, _ptr(out)))
        return out

    def Reserve(self, pages: int) -> None:
        check(self._lib.qr_mla_reserve(self._h, pages))

    def Append(self, layer, pos, latent) -> None:
        row = np.ascontiguousarray(latent, dtype=np.float32).reshape(-1)
        check(self._lib.qr_mla_append(self._h, layer, pos, _ptr(row), row.size))

    def AppendRange(self, layer, pos0, rows, src_dtype="f32") -> None:
        code = dtype_code(src_dtype)
        r = _host_rows(rows, code)
        n = r.size // self.LatentDim
        if r.size != n * self.LatentDim:
            raise ValueError("rows must be [n, kv_lora + rope]")
        check(self._lib.qr_mla_append_range(self._h, layer, pos0, n, _ptr(r), code))

    def AppendRangeDev(self, layer, pos0, rows, src_dtype="f32", stream=None) -> None:
        code = dtype_code(src_dtype)
        n = _rows_of(rows, self.LatentDim, "latent rows")
        rp = _dev_tensor(rows, n * self.LatentDim, code, "latent rows")
        check(self._lib.qr_mla_append_range_dev(self._h, layer, pos0, n, rp, code, _stream_ptr(stream)))

    def Reset(self) -> None:
        check(self._lib.qr_mla_reset(self._h))

    def Truncate(self, length) -> None:
        check(self._lib.qr_mla_truncate(self._h, length))

    def _split(self):
        """(kv_lora, rope); before SetRope on a cache made from its latent width alone, the
        whole row -- the library then rejects attention calls until the split is set."""
        return (self.KvLora, self.Rope) if self.Rope is not None else (self.LatentDim, 0)

    def AbsorbedAttention(self, layer, pos, q_tilde, q_rope, scale) -> np.ndarray:
        """u [heads, kv_lora] = softmax(q~.c + q_rope.k_pe) . c over positions 0..pos."""
        kv_lora, rope = self._split()
        qt = np.ascontiguousarray(q_tilde, dtype=np.float32)
        heads = qt.size // kv_lora
        qr = np.ascontiguousarray(q_rope if rope else np.zeros(1), dtype=np.float32)
        if rope and qr.size != heads * rope:
            raise ValueError("q_rope must be [heads, rope]")
        u = np.empty((heads, kv_lora), np.float32)
        check(self._lib.qr_mla_attention(self._h, layer, pos, heads, _ptr(qt), _ptr(qr), scale, _ptr(u)))
        return u

    def AttendAbsorbed(self, layer, pos, q, kvb, nope, vdim) -> np.ndarray:
        """MlaLayer's absorbed block (StreamingEngine.cs:508-577) for one token: q [heads,
        nope+rope] (rope part rotated), kvb a Weight of [heads*(nope+vdim), kv_lora].
        Returns the attention output [heads, vdim]."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        heads = q.size // (nope + self._split()[1])
        out = np.empty((heads, vdim), np.float32)
        check(self._lib.qr_mla_attend_absorbed(self._h, layer, pos, heads, nope, vdim, _ptr(q), kvb.handle,
                                               _ptr(out)))
        return out

    def AttendAbsorbedDev(self, layer, pos, q, kvb, fmt, nope, vdim, out, stream=None) -> None:
        """Device form: q, out torch tensors on the GPU; kvb a Weight or a uint8 device tensor
        of rows in format `fmt`."""
        f32 = _lib.DTYPE_F32
        rope = self._split()[1]
        heads = _rows_of(q, nope + rope, "q")
        qp = _dev_tensor(q, heads * (nope + rope), f32, "q")
        op = _dev_tensor(out, heads * vdim, f32, "out")
        check(self._lib.qr_mla_attend_absorbed_dev(self._h, layer, pos, heads, nope, vdim, qp, _dev_ptr(kvb), fmt,
                                                   op, _stream_ptr(stream)))

    def AbsorbedAttentionDev(self, layer, pos, q_tilde, q_rope, u, scale, stream=None) -> None:
        f32 = _lib.DTYPE_F32
        kv_lora, rope = self._split()
        heads = _rows_of(q_tilde, kv_lora, "q_tilde")
        qt = _dev_tensor(q_tilde, heads * kv_lora, f32, "q_tilde")
        qr_ptr = _dev_tensor(q_rope, heads * rope, f32, "q_rope", allow_none=rope == 0)
        up = _dev_tensor(u, heads * kv_lora, f32, "u")
        check(self._lib.qr_mla_attention_dev(self._h, layer, pos, heads, qt, qr_ptr, scale, up,
                                             _stream_ptr(stream)))

    # ---- device-position forms (graph-capturable steps; pages reserved before capture)
    def AppendStepDev(self, layer, pos0_dev, rows, src_dtype="f32", stream=None) -> None:
        """AppendRangeDev at the positions pos0_dev[0] .. + n - 1 read on the GPU (int32 [1]);
        their pages are claimed on the device."""
        code = dtype_code(src_dtype)
        n = _rows_of(rows, self.LatentDim, "latent rows")
        pp = _dev_int32(pos0_dev, 1, "pos0")
        rp = _dev_tensor(rows, n * self.LatentDim, code, "latent rows")
        check(self._lib.qr_mla_append_step_dev(self._h, layer, n, pp, rp, code, _stream_ptr(stream)))

    def AbsorbedAttentionStepDev(self, layer, pos_dev, q_tilde, q_rope, u, scale, stream=None) -> None:
        """AbsorbedAttentionDev at the position read on the GPU from pos_dev (int32 [1])."""
        f32 = _lib.DTYPE_F32
        kv_lora, rope = self._split()
        heads = _rows_of(q_tilde, kv_lora, "q_tilde")
        pp = _dev_int32(pos_dev, 1, "pos")
        qt = _dev_tensor(q_tilde, heads * kv_lora, f32, "q_tilde")
        qr_ptr = _dev_tensor(q_rope, heads * rope, f32, "q_rope", allow_none=rope == 0)
        up = _dev_tensor(u, heads * kv_lora, f32, "u")
        check(self._lib.qr_mla_attention_step_dev(self._h, layer, pp, heads, qt, qr_ptr, scale, up,
                                                  _stream_ptr(stream)))

    def AttendAbsorbedStepDev(self, layer, pos_dev, q, kvb, fmt, nope, vdim, out, stream=None) -> None:
        """AttendAbsorbedDev at the position read on the GPU from pos_dev (int32 [1])."""
        f32 = _lib.DTYPE_F32
        rope = self._split()[1]
        heads = _rows_of(q, nope + rope, "q")
        pp = _dev_int32(pos_dev, 1, "pos")
        qp = _dev_tensor(q, heads * (nope + rope), f32, "q")
        op = _dev_tensor(out, heads * vdim, f32, "out")
        check(self._lib.qr_mla_attend_absorbed_step_dev(self._h, layer, pp, heads, nope, vdim, qp, _dev_ptr(kvb),
                                                        fmt, op, _stream_ptr(stream)))
