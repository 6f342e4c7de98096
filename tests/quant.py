"""Block encoders for test weights (QuantFormat rows, Dtypes.cs:6-50).

These write valid blocks of each format the kvb decoders cover, from the block
layouts alone: a weight index maps to the byte and bit field that hold it.  They
are not the reference's quantizers (BlockQuantizer.cs searches scales more
carefully); the tests use them to produce weight rows and to pin the decoders by
encode -> decode round trips, so any consistent encoding serves.

Layouts (byte offsets inside one block):
  Q4_0  20 B / 32 w : f16 d @0, nibbles @2 (weight i low nibble of byte i, weight
                      i+16 high nibble), 2 pad bytes; w = d * (q - 8)
  Q8_0  34 B / 32 w : f16 d @0, int8 @2; w = d * q
  Q4_K 144 B / 256 w: f16 d @0, f16 dmin @2, 12 packed 6-bit scale/min bytes @4,
                      nibbles @16 (sub-blocks 2p, 2p+1 share bytes 32p..32p+31,
                      low / high nibble); w = (d*sc_j) * q - dmin*m_j
  Q6_K 210 B / 256 w: low nibbles @0 (128 B), 2-bit high parts @128 (64 B),
                      int8 scales @192 (16), f16 d @208; w = (d*sc) * (q - 32)
"""
from __future__ import annotations

import numpy as np

FMT = {"F32": 0, "F16": 1, "BF16": 2, "Q4_0": 3, "Q8_0": 4, "Q4_K": 6, "Q6_K": 7}
BLOCK = {0: (1, 4), 1: (1, 2), 2: (1, 2), 3: (32, 20), 4: (32, 34), 6: (256, 144), 7: (256, 210)}


def row_bytes(fmt, n):
    bs, bb = BLOCK[fmt]
    assert n % bs == 0
    return n // bs * bb


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16)


def _put_f16(blk, off, v):
    blk[..., off:off + 2] = _f16(v).reshape(-1, 1).view(np.uint8).reshape(blk.shape[:-1] + (2,))


# ---- placement maps: weight index inside a block -> where its bits live -------

def q4k_nibble_slot(w):
    """Q4_K weight w (0..255) -> (byte offset of its nibble, high nibble?, sub-block)."""
    sub, i = w // 32, w % 32
    return 16 + (sub // 2) * 32 + i, sub % 2 == 1, sub


def q6k_slots(w):
    """Q6_K weight w -> (low-nibble byte, high nibble?, high-bits byte, shift, scale byte)."""
    half, r = w // 128, w % 128
    m, l = r // 32, r % 32
    ql = half * 64 + l + (32 if m % 2 else 0)
    qh = 128 + half * 32 + l
    sc = 192 + 8 * half + l // 16 + 2 * m
    return ql, m >= 2, qh, 2 * m, sc


def pack_scale_min_k4(sc, mn):
    """Inverse of the 6-bit scale/min packing (BlockDequantizer.cs:155-166): 8 pairs -> 12 bytes."""
    out = np.zeros(12, np.uint8)
    for j in range(8):
        s, m = int(sc[j]), int(mn[j])
        assert 0 <= s < 64 and 0 <= m < 64
        if j < 4:
            out[j] |= s & 63
            out[j + 4] |= m & 63
        else:
            out[j + 4] |= (s & 0xF) | ((m & 0xF) << 4)
            out[j - 4] |= (s >> 4) << 6
            out[j] |= (m >> 4) << 6
    return out


# ---- block builders from integer fields ---------------------------------------

def build_q4k_block(d, dmin, sc, mn, q):
    blk = np.zeros(144, np.uint8)
    blk[0:2] = _f16(d).reshape(1).view(np.uint8)
    blk[2:4] = _f16(dmin).reshape(1).view(np.uint8)
    blk[4:16] = pack_scale_min_k4(sc, mn)
    for w in range(256):
        off, hi, _ = q4k_nibble_slot(w)
        blk[off] |= (int(q[w]) & 0xF) << (4 if hi else 0)
    return blk


def build_q6k_block(d, sc, q):
    """q: 256 values in [0, 63]; sc: 16 int8 scales."""
    blk = np.zeros(210, np.uint8)
    for w in range(256):
        ql, hi, qh, sh, _ = q6k_slots(w)
        v = int(q[w])
        blk[ql] |= (v & 0xF) << (4 if hi else 0)
        blk[qh] |= ((v >> 4) & 3) << sh
    blk[192:208] = np.asarray(sc, np.int8).view(np.uint8)
    blk[208:210] = _f16(d).reshape(1).view(np.uint8)
    return blk


def q6k_scale_index(w):
    return q6k_slots(w)[4] - 192


# ---- encoders from fp32 rows ----------------------------------------------------

def _round(x):
    return np.floor(x + 0.5)


def quantize(fmt, x):
    """fp32 [rows][n] -> uint8 [rows][row_bytes] in format fmt (vectorised over blocks)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, n = x.shape
    if fmt == 0:
        return x.view(np.uint8).reshape(rows, -1).copy()
    if fmt == 1:
        return x.astype(np.float16).view(np.uint8).reshape(rows, -1).copy()
    if fmt == 2:
        from oracle import oracle
        return oracle.f32_to_bf16(x).view(np.uint8).reshape(rows, -1).copy()
    bs, bb = BLOCK[fmt]
    xb = x.reshape(rows * (n // bs), bs).astype(np.float64)
    if fmt == 4:
        out = np.zeros((xb.shape[0], bb), np.uint8)
        d = _f16(np.abs(xb).max(-1) / 127.0).astype(np.float64)
        q = np.clip(_round(xb / np.where(d > 0, d, 1)[:, None]), -128, 127).astype(np.int8)
        _put_f16(out, 0, d)
        out[:, 2:34] = q.view(np.uint8)
    elif fmt == 3:
        out = np.zeros((xb.shape[0], bb), np.uint8)
        d = _f16(np.abs(xb).max(-1) / 8.0).astype(np.float64)
        q = np.clip(_round(xb / np.where(d > 0, d, 1)[:, None]) + 8, 0, 15).astype(np.uint8)
        _put_f16(out, 0, d)
        out[:, 2:18] = q[:, :16] | (q[:, 16:] << 4)
    elif fmt == 6:
        sub = xb.reshape(-1, 8, 32)
        lo = np.minimum(sub.min(-1), 0.0)
        scale = (sub.max(-1) - lo) / 15.0
        d = _f16(np.maximum(scale.max(-1), 1e-8) / 63.0).astype(np.float64)
        dmin = _f16(np.maximum((-lo).max(-1), 1e-8) / 63.0).astype(np.float64)
        sc = np.clip(_round(scale / d[:, None]), 1, 63).astype(np.int64)
        mn = np.clip(_round(-lo / dmin[:, None]), 0, 63).astype(np.int64)
        a = d[:, None] * sc
        m = dmin[:, None] * mn
        q = np.clip(_round((sub + m[..., None]) / a[..., None]), 0, 15).astype(np.int64)
        out = pack_q4k(d, dmin, sc, mn, q.reshape(-1, 256))
    elif fmt == 7:
        g = xb.reshape(-1, 2, 4, 2, 16)          # [block][half][m][l // 16][l % 16]
        amax = np.abs(g).max(-1) / 31.0          # 16 groups, scale byte 8*half + 2*m + l//16
        d = _f16(np.maximum(amax.reshape(-1, 16).max(-1), 1e-8) / 127.0).astype(np.float64)
        sc = np.clip(_round(amax / d[:, None, None, None]), 1, 127).astype(np.int64)
        q = np.clip(_round(g / (d[:, None, None, None, None] * sc[..., None])) + 32, 0, 63).astype(np.int64)
        out = pack_q6k(d, sc.reshape(-1, 16), q.reshape(-1, 256))
    else:
        raise ValueError(fmt)
    return out.reshape(rows, -1)


def pack_q4k(d, dmin, sc, mn, q):
    """Vectorised Q4_K blocks: d, dmin [B]; sc, mn [B][8] in [0, 63]; q [B][256] in [0, 15]."""
    B = q.shape[0]
    out = np.zeros((B, 144), np.uint8)
    _put_f16(out, 0, d)
    _put_f16(out, 2, dmin)
    out[:, 4:8] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    out[:, 12:16] = (sc[:, 4:8] & 0xF) | ((mn[:, 4:8] & 0xF) << 4)
    qs = q.reshape(B, 4, 2, 32)
    out[:, 16:144] = (qs[:, :, 0, :] | (qs[:, :, 1, :] << 4)).reshape(B, 128)
    return out


def pack_q6k(d, sc, q):
    """Vectorised Q6_K blocks: d [B]; sc [B][16] int8 in scale-byte order; q [B][256] in [0, 63]."""
    B = q.shape[0]
    out = np.zeros((B, 210), np.uint8)
    qq = q.reshape(B, 2, 4, 32)                  # [half][m][l]
    lo, hi = qq & 0xF, qq >> 4
    ql = np.stack([lo[:, :, 0] | (lo[:, :, 2] << 4), lo[:, :, 1] | (lo[:, :, 3] << 4)], axis=2)
    out[:, 0:128] = ql.reshape(B, 128)
    out[:, 128:192] = (hi[:, :, 0] | (hi[:, :, 1] << 2) | (hi[:, :, 2] << 4) | (hi[:, :, 3] << 6)).reshape(B, 64)
    out[:, 192:208] = np.asarray(sc, np.int64).astype(np.int8).view(np.uint8)
    _put_f16(out, 208, d)
    return out


def random_rows(fmt, rows, n, seed, std=0.05):
    """Seeded N(0, std^2) weights encoded in fmt: (uint8 rows, decoded via the oracle)."""
    from oracle import oracle
    x = np.random.default_rng(seed).standard_normal((rows, n)).astype(np.float32) * np.float32(std)
    raw = quantize(fmt, x)
    return raw, oracle.dequant_rows(fmt, raw, n)
