"""numpy front end of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: this module is the checker.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import it; the product
library never does.  Every function forwards to the C restatement in
qr_oracle.c, which cites the reference lines it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i, _l, _f, _d = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double


def build() -> None:
    """Compile the oracle in place (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "qro_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "qro_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "qro_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "qro_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
            "qro_f16_to_f32_n": (None, [_u16p, _f32p, _l]),
            "qro_f32_to_f16_n": (None, [_f32p, _u16p, _l]),
            "qro_bf16_to_f32_n": (None, [_u16p, _f32p, _l]),
            "qro_f32_to_bf16_n": (None, [_f32p, _u16p, _l]),
            "qro_dot_f32": (ctypes.c_float, [_f32p, _f32p, _i]),
            "qro_axpy_f32": (None, [_f32p, _f32p, _f, _i]),
            "qro_softmax": (None, [_f32p, _i]),
            "qro_build_cos_sin": (None, [_l, _i, _f, _f32p]),
            "qro_rope_rows": (None, [_f32p, _l, _i, _i, _l, _f]),
            "qro_kv_attention": (None, [_f32p, _f32p, _i, _i, _i, _i, _f32p, _f32p, _f, _f32p]),
            "qro_kv_attention_f64": (None, [_f32p, _f32p, _i, _i, _i, _i, _f32p, _f64p, _d]),
            "qro_mla_attention": (None, [_f32p, _i, _i, _i, _i, _f32p, _f32p, _f, _f32p, _f32p]),
            "qro_mla_attention_f64": (None, [_f32p, _i, _i, _i, _i, _f32p, _f32p, _d, _f64p]),
            "qro_mla_q_absorb": (None, [_f32p, _f32p, _i, _i, _i, _i, _i, _f32p]),
            "qro_mla_wuv": (None, [_f32p, _f32p, _i, _i, _i, _i, _f32p]),
            "qro_mla_expanded_f64": (None, [_f32p, _f32p, _f32p, _i, _i, _i, _i, _i, _i, _d, _f64p]),
            "qro_row_bytes": (ctypes.c_long, [_i, _l]),
            "qro_dequant_row": (ctypes.c_int, [_i, _u8p, _l, _f32p]),
            "qro_dot_row": (ctypes.c_float, [_i, _u8p, _f32p, _i]),
            "qro_matvec": (ctypes.c_int, [_i, _u8p, _l, _i, _f32p, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- codecs
def f16_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().qro_f16_to_f32_n(b.reshape(-1), out.reshape(-1), b.size)
    return out


def f32_to_f16(x):
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().qro_f32_to_f16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().qro_bf16_to_f32_n(b.reshape(-1), out.reshape(-1), b.size)
    return out


def f32_to_bf16(x):
    x = _c32(x)
    out = np.empty(x.shape, np.uint16)
    lib().qro_f32_to_bf16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


# ---------------------------------------------------------------- primitives
def dot_f32(a, b):
    a, b = _c32(a), _c32(b)
    return float(lib().qro_dot_f32(a, b, a.size))


def axpy_f32(x, y, alpha):
    x = _c32(x)
    y = _c32(y).copy()
    lib().qro_axpy_f32(x, y, alpha, x.size)
    return y


def softmax(x):
    x = _c32(x).copy()
    lib().qro_softmax(x, x.size)
    return x


def build_cos_sin(pos, head_dim, theta):
    row = np.empty(head_dim, np.float32)
    lib().qro_build_cos_sin(pos, head_dim, theta, row)
    return row


def rope_rows(x, head_dim, pos0, theta):
    """RoPE (TransformerOps.cs:56-88) on rows of `x` [rows, width]; row r sits at pos0 + r."""
    x = _c32(x).copy()
    rows, width = x.shape
    lib().qro_rope_rows(x.reshape(-1), rows, width, head_dim, pos0, theta)
    return x


# ---------------------------------------------------------------- attention
def kv_attention(K, V, q, heads, kv_heads, head_dim, scale):
    """PagedKvCache.Attention restatement.  K, V: [seq, kv_heads*head_dim] fp32 rows
    0..pos; q: [heads*head_dim].  Returns attn [heads*head_dim] fp32."""
    K, V, q = _c32(K), _c32(V), _c32(q).reshape(-1)
    seq = K.shape[0]
    out = np.empty(heads * head_dim, np.float32)
    scratch = np.empty(max(heads * seq, 1), np.float32)
    lib().qro_kv_attention(K.reshape(-1), V.reshape(-1), seq, heads, kv_heads, head_dim, q, out,
                           scale, scratch)
    return out


def kv_attention_f64(K, V, q, heads, kv_heads, head_dim, scale):
    K, V, q = _c32(K), _c32(V), _c32(q).reshape(-1)
    out = np.empty(heads * head_dim, np.float64)
    lib().qro_kv_attention_f64(K.reshape(-1), V.reshape(-1), K.shape[0], heads, kv_heads,
                               head_dim, q, out, scale)
    return out


def mla_attention(lat, q_tilde, q_rope, kv_lora, rope, scale):
    """StreamingEngine.cs:531-568 score -> softmax -> latent sum.  lat [seq, kv_lora+rope],
    q_tilde [heads, kv_lora], q_rope [heads, rope] -> u [heads, kv_lora]."""
    lat, qt = _c32(lat), _c32(q_tilde)
    heads = qt.shape[0]
    qr = _c32(q_rope) if rope > 0 else np.zeros((heads, 1), np.float32)
    seq = lat.shape[0]
    u = np.empty((heads, kv_lora), np.float32)
    scratch = np.empty(max(seq, 1), np.float32)
    lib().qro_mla_attention(lat.reshape(-1), seq, kv_lora, rope, heads, qt.reshape(-1),
                            qr.reshape(-1), scale, u.reshape(-1), scratch)
    return u


def mla_attention_f64(lat, q_tilde, q_rope, kv_lora, rope, scale):
    lat, qt = _c32(lat), _c32(q_tilde)
    heads = qt.shape[0]
    qr = _c32(q_rope) if rope > 0 else np.zeros((heads, 1), np.float32)
    u = np.empty((heads, kv_lora), np.float64)
    lib().qro_mla_attention_f64(lat.reshape(-1), lat.shape[0], kv_lora, rope, heads,
                                qt.reshape(-1), qr.reshape(-1), scale, u.reshape(-1))
    return u


def mla_q_absorb(q, kvb, heads, nope, rope, vdim, kv_lora):
    q, kvb = _c32(q), _c32(kvb)
    out = np.empty((heads, kv_lora), np.float32)
    lib().qro_mla_q_absorb(q.reshape(-1), kvb.reshape(-1), heads, nope, rope, vdim, kv_lora,
                           out.reshape(-1))
    return out


def mla_wuv(u, kvb, heads, nope, vdim, kv_lora):
    u, kvb = _c32(u), _c32(kvb)
    out = np.empty((heads, vdim), np.float32)
    lib().qro_mla_wuv(u.reshape(-1), kvb.reshape(-1), heads, nope, vdim, kv_lora, out.reshape(-1))
    return out


def mla_expanded_f64(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale):
    q, kvb, lat = _c32(q), _c32(kvb), _c32(lat)
    out = np.empty((heads, vdim), np.float64)
    lib().qro_mla_expanded_f64(q.reshape(-1), kvb.reshape(-1), lat.reshape(-1), lat.shape[0],
                               heads, nope, rope, vdim, kv_lora, scale, out.reshape(-1))
    return out


# QuantFormat values (Dtypes.cs:6-26) that the decoders cover.
FMT = {"F32": 0, "F16": 1, "BF16": 2, "Q4_0": 3, "Q8_0": 4, "Q4_K": 6, "Q6_K": 7}


def row_bytes(fmt, n):
    """Bytes of one row of n weights (Dtypes.cs:38-50); ValueError if not whole blocks."""
    r = lib().qro_row_bytes(int(fmt), int(n))
    if r < 0:
        raise ValueError(f"format {fmt} cannot hold a row of {n} weights")
    return r


def dequant_rows(fmt, raw, n):
    """BlockDequantizer.Dequantize on every row of raw (uint8 [rows][row_bytes]) -> fp32 [rows][n]."""
    rb = row_bytes(fmt, n)
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, rb)
    out = np.empty((raw.shape[0], n), np.float32)
    for r in range(raw.shape[0]):
        if lib().qro_dequant_row(int(fmt), raw[r], n, out[r]) != 0:
            raise ValueError(f"format {fmt} unsupported")
    return out


def matvec(fmt, raw, cols, x):
    """DotKernels.MatVec: y[r] = DotRow(fmt, row r of raw, x) in the reference's per-format order."""
    rb = row_bytes(fmt, cols)
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, rb)
    x = _c32(x).reshape(-1)
    y = np.empty(raw.shape[0], np.float32)
    if lib().qro_matvec(int(fmt), raw.reshape(-1), raw.shape[0], cols, x, y) != 0:
        raise ValueError(f"format {fmt} unsupported")
    return y
