"""Pins the CPU oracle before it is trusted as the checker.

Each check is one the oracle could fail: the reference's own known-answer and
invariant tests (tests/QuantRunner.Tests/Program.cs, Cli/Commands.cs
selftests), library routines (numpy/torch float conversions, fp64 formulas),
and closed forms built so that a dropped term, a wrong lane order, an FMA in
place of multiply-then-add, or a wrong GQA map gives a different number.
"""
import math

import numpy as np
import pytest

from oracle import oracle, paging
from tests.util import assert_close, normal

F32 = np.float32


# ------------------------------------------------------------------ 16-bit codecs
def test_f16_known_answers():
    """Tests/Program.cs:60-70 (F16Conv)."""
    L = oracle.lib()
    assert L.qro_f16_to_f32(0) == 0.0
    neg0 = L.qro_f16_to_f32(0x8000)
    assert neg0 == 0.0 and math.copysign(1.0, neg0) < 0
    assert L.qro_f16_to_f32(0x3C00) == 1.0
    assert L.qro_f16_to_f32(0xBC00) == -1.0
    assert L.qro_f16_to_f32(0x7BFF) == 65504.0
    assert math.isinf(L.qro_f16_to_f32(0x7C00)) and L.qro_f16_to_f32(0x7C00) > 0
    assert abs(L.qro_f16_to_f32(0x0001) - 5.9604645e-8) <= 1e-13


def test_f16_decode_all_patterns_match_numpy():
    """F16ToFloat (Dtypes.cs:76-97) is exact widening: equal to numpy for all 65536 patterns."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = oracle.f16_to_f32(bits).view(np.uint32)
    ref = bits.view(np.float16).astype(np.float32).view(np.uint32)
    finite = (bits & 0x7C00) != 0x7C00
    assert np.array_equal(ours[finite], ref[finite])
    # inf/nan: sign | 0x7F800000 | man << 13
    man = (bits[~finite].astype(np.uint32) & 0x3FF) << 13
    sign = (bits[~finite].astype(np.uint32) & 0x8000) << 16
    assert np.array_equal(ours[~finite], sign | 0x7F800000 | man)


def test_f16_encode_round_trip_tolerance():
    """Tests/Program.cs:71-82: round trip within 0.05% (normal) / 2^-24 abs (subnormal)."""
    rng = np.random.default_rng(1)
    v = ((rng.random(100000) * 2 - 1) * np.power(2.0, rng.integers(-14, 15, 100000))).astype(F32)
    back = oracle.f16_to_f32(oracle.f32_to_f16(v))
    sub = np.abs(v) < 6.1e-5
    tol = np.where(sub, 6e-8, np.abs(v) * 0.0005 + 1e-30)
    assert np.all(np.abs(back - v) <= tol)


def test_f16_encode_matches_rne_except_normal_ties():
    """FloatToF16 adds half an ulp and truncates in the normal range (Dtypes.cs:111-113):
    equal to round-nearest-even except at exact ties, which go away from zero."""
    rng = np.random.default_rng(2)
    v = (rng.standard_normal(200000) * 100).astype(F32)
    ours = oracle.f32_to_f16(v)
    rne = v.astype(np.float16).view(np.uint16)
    man = v.view(np.uint32) & 0x1FFF
    tie = man == 0x1000
    assert np.array_equal(ours[~tie], rne[~tie])
    # constructed ties: 1 + 2^-11 sits halfway between 0x3C00 and 0x3C01
    t = np.array([1 + 2 ** -11, -(1 + 2 ** -11), 1 + 3 * 2 ** -11], F32)
    assert list(oracle.f32_to_f16(t)) == [0x3C01, 0xBC01, 0x3C02]
    assert list(t.astype(np.float16).view(np.uint16)) == [0x3C00, 0xBC00, 0x3C02]
    # subnormal range is round-nearest-even: 2^-25 ties to 0, 3*2^-25 ties to 2*2^-24
    s = np.array([2 ** -25, 3 * 2 ** -25, 2 ** -26], F32)
    assert list(oracle.f32_to_f16(s)) == [0x0000, 0x0002, 0x0000]
    # overflow and specials
    sp = np.array([70000.0, -np.inf, np.nan, 65520.0], F32)
    out = oracle.f32_to_f16(sp)
    assert out[0] == 0x7C00 and out[1] == 0xFC00 and out[2] == 0x7E00 and out[3] == 0x7C00


def test_bf16_known_answers_and_rne():
    """Tests/Program.cs:85-92 (Bf16Conv) plus RNE (Dtypes.cs:132-139) against torch."""
    torch = pytest.importorskip("torch")
    L = oracle.lib()
    assert L.qro_bf16_to_f32(L.qro_f32_to_bf16(1.0)) == 1.0
    assert L.qro_bf16_to_f32(L.qro_f32_to_bf16(-2.5)) == -2.5
    pi = np.float32(math.pi)
    assert abs(L.qro_bf16_to_f32(L.qro_f32_to_bf16(pi)) - pi) / pi <= 0.01
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(100000) * 50).astype(F32)
    ties = np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8)], F32)  # halfway cases
    v = np.concatenate([v, ties])
    ours = oracle.f32_to_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    assert np.array_equal(oracle.bf16_to_f32(bits).view(np.uint32), bits.astype(np.uint32) << 16)


# ------------------------------------------------------------------ primitives
def test_dot_lane_order_closed_forms():
    """DotF32 (SimdMath.cs:34-53): 8 lane accumulators, lanes summed 0..7, then the tail."""
    a = np.zeros(16, F32)
    a[0], a[1:8], a[8] = 1e8, 1.0, -1e8
    # lanes: lane0 = 1e8 + -1e8 = 0, lanes 1..7 = 1 -> 7 (a sequential sum gives 0)
    assert oracle.dot_f32(a, np.ones(16, F32)) == 7.0
    b = np.zeros(9, F32)
    b[0], b[1], b[8] = 1e8, 1.0, -1e8
    # HSum absorbs the 1 (1e8 + 1 == 1e8 in fp32) before the tail -1e8 -> 0
    assert oracle.dot_f32(b, np.ones(9, F32)) == 0.0
    c = np.array([1e8, 1.0, -1e8], F32)  # n < 8: plain sequential sum
    assert oracle.dot_f32(c, np.ones(3, F32)) == 0.0
    d = np.array([1.0, 1e8, -1e8], F32)
    assert oracle.dot_f32(d, np.ones(3, F32)) == 0.0


def test_dot_and_axpy_do_not_fuse():
    """Multiply then add, separately rounded: (1+2^-12)^2 - (1+2^-11) is 0 without FMA, 2^-24 with."""
    x = F32(1 + 2 ** -12)
    y = F32(-(1 + 2 ** -11))
    a = np.array([x] + [0] * 7, F32)
    b = np.array([x] + [0] * 7, F32)
    assert oracle.dot_f32(np.concatenate([a, [y]]).astype(F32), np.concatenate([b, [1]]).astype(F32)) == 0.0
    out = oracle.axpy_f32(np.full(8, x, F32), np.full(8, y, F32), float(x))
    assert np.all(out == 0.0)
    out3 = oracle.axpy_f32(np.full(3, x, F32), np.full(3, y, F32), float(x))  # scalar tail
    assert np.all(out3 == 0.0)


def test_dot_matches_fp64():
    for n in (5, 16, 64, 128, 576):
        a, b = normal(10 + n, n), normal(20 + n, n)
        assert abs(oracle.dot_f32(a, b) - float(a.astype(np.float64) @ b)) <= 1e-4 * math.sqrt(n)


def test_softmax_closed_forms():
    """TransformerOps.Softmax (:92-107)."""
    assert np.array_equal(oracle.softmax(np.array([3.5], F32)), np.array([1.0], F32))
    np.testing.assert_allclose(oracle.softmax(np.zeros(10, F32)), np.full(10, 0.1, F32), rtol=1e-7)
    np.testing.assert_allclose(oracle.softmax(np.array([0, math.log(2)], F32)), [1 / 3, 2 / 3], rtol=1e-6)
    x = normal(5, 1000)
    np.testing.assert_allclose(oracle.softmax(x), oracle.softmax(x + 1000), rtol=1e-4, atol=1e-9)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(oracle.softmax(x), e / e.sum(), rtol=1e-5)


def test_rope_norm_preserved_and_identity_at_zero():
    """Tests/Program.cs:282-306 (RopeTest, theta 10000, pos 123) and pos 0 == identity."""
    rng = np.random.default_rng(9)
    q = (rng.random(128) - 0.5).astype(F32)
    out = oracle.rope_rows(q.reshape(1, -1), 64, 123, 10000.0).reshape(-1)
    for h in range(2):
        before = float(np.sum(q[h * 64:(h + 1) * 64].astype(np.float64) ** 2))
        after = float(np.sum(out[h * 64:(h + 1) * 64].astype(np.float64) ** 2))
        assert abs(before - after) / before <= 1e-4
    assert np.array_equal(oracle.rope_rows(q.reshape(1, -1), 64, 0, 10000.0).reshape(-1), q)


def test_rope_matches_fp64_rotation():
    x = normal(11, (4, 2 * 128))
    out = oracle.rope_rows(x, 128, 32764, 500000.0)
    D, half = 128, 64
    i = np.arange(half, dtype=np.float64)
    for r in range(4):
        ang = (32764 + r) * np.power(500000.0, -2 * i / D)
        c, s = np.cos(ang), np.sin(ang)
        for h in range(2):
            v = x[r, h * D:(h + 1) * D].astype(np.float64)
            want = np.concatenate([v[:half] * c - v[half:] * s, v[:half] * s + v[half:] * c])
            # fp32 angles at ~3e4 rad carry ~2e-3 rad of rounding: compare loosely
            np.testing.assert_allclose(out[r, h * D:(h + 1) * D], want, atol=2e-2)


# ------------------------------------------------------------------ GQA decode attention
def _kvcache_test_rows(kv_dim):
    i = np.arange(kv_dim)
    return np.sin(i).astype(F32), np.cos(i).astype(F32)


@pytest.mark.parametrize("heads,kv_heads,seq", [(4, 2, 700), (2, 2, 600)])
def test_kv_attention_reference_invariants(heads, kv_heads, seq):
    """Tests/Program.cs:242-280 and Cli/Commands.cs:3037-3065: identical rows ->
    uniform softmax -> attn == V of the mapped kv head, for q = 0 and q = 1."""
    D = 16
    k, v = _kvcache_test_rows(kv_heads * D)
    K = np.tile(k, (seq, 1))
    V = np.tile(v, (seq, 1))
    for qv in (0.0, 1.0):
        q = np.full(heads * D, qv, F32)
        out = oracle.kv_attention(K, V, q, heads, kv_heads, D, 0.25)
        for h in range(heads):
            kvh = h * kv_heads // heads
            assert np.all(np.abs(out[h * D:(h + 1) * D] - v[kvh * D:(kvh + 1) * D]) <= 1e-4)


@pytest.mark.parametrize("heads,kv_heads", [(8, 2), (6, 4), (5, 3), (4, 4)])
def test_kv_attention_gqa_map(heads, kv_heads):
    """kvh = h*kv_heads/heads (PagedKvCache.cs:103): V rows constant per kv head."""
    D, seq = 16, 40
    K = normal(1, (seq, kv_heads * D))
    V = np.zeros((seq, kv_heads * D), F32)
    for g in range(kv_heads):
        V[:, g * D:(g + 1) * D] = g + 1
    out = oracle.kv_attention(K, V, normal(2, heads * D), heads, kv_heads, D, 0.25)
    for h in range(heads):
        np.testing.assert_allclose(out[h * D:(h + 1) * D], h * kv_heads // heads + 1, rtol=1e-6)


def test_kv_attention_single_position_is_exact():
    K, V = normal(3, (1, 2 * 64)), normal(4, (1, 2 * 64))
    out = oracle.kv_attention(K, V, normal(5, 8 * 64), 8, 2, 64, 0.125)
    for h in range(8):
        assert np.array_equal(out[h * 64:(h + 1) * 64], V[0, (h // 4) * 64:(h // 4 + 1) * 64])


@pytest.mark.parametrize("heads,kv_heads,D,seq", [(8, 2, 64, 512), (6, 4, 16, 300), (32, 8, 128, 1000)])
def test_kv_attention_matches_fp64(heads, kv_heads, D, seq):
    K, V = normal(6, (seq, kv_heads * D)), normal(7, (seq, kv_heads * D))
    q = normal(8, heads * D)
    s = 1 / math.sqrt(D)
    assert_close(oracle.kv_attention(K, V, q, heads, kv_heads, D, s),
                 oracle.kv_attention_f64(K, V, q, heads, kv_heads, D, s), 1e-5, 1e-5, "oracle vs fp64")


# ------------------------------------------------------------------ MLA
def _absorbed(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale):
    qt = oracle.mla_q_absorb(q, kvb, heads, nope, rope, vdim, kv_lora)
    qk = nope + rope
    qr = q.reshape(heads, qk)[:, nope:]
    u = oracle.mla_attention(lat, qt, qr, kv_lora, rope, scale)
    return oracle.mla_wuv(u, kvb, heads, nope, vdim, kv_lora)


def test_mla_absorbed_equals_expanded_reference_shape():
    """Cli/Commands.cs:2065-2152: H4 kvLora8 nope4 v4 seq10 rope0, U[-1,1], <= 1e-4 vs fp64."""
    heads, kv_lora, nope, vdim, seq = 4, 8, 4, 4, 10
    rng = np.random.default_rng(29)
    R = lambda n: (rng.random(n) * 2 - 1).astype(F32)  # noqa: E731
    q = R(heads * nope)
    kvb = R(heads * (nope + vdim) * kv_lora)
    lat = R(seq * kv_lora).reshape(seq, kv_lora)
    scale = 1 / math.sqrt(nope)
    got = _absorbed(q, kvb, lat, heads, nope, 0, vdim, kv_lora, scale)
    want = oracle.mla_expanded_f64(q, kvb, lat, heads, nope, 0, vdim, kv_lora, scale)
    assert np.max(np.abs(got - want)) <= 1e-4


def test_mla_absorbed_equals_expanded_with_rope():
    heads, kv_lora, nope, rope, vdim, seq = 4, 64, 16, 16, 16, 300
    rng = np.random.default_rng(30)
    R = lambda n: (rng.random(n) * 2 - 1).astype(F32)  # noqa: E731
    q = R(heads * (nope + rope))
    kvb = R(heads * (nope + vdim) * kv_lora)
    lat = R(seq * (kv_lora + rope)).reshape(seq, kv_lora + rope)
    scale = 1 / math.sqrt(nope + rope)
    got = _absorbed(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale)
    want = oracle.mla_expanded_f64(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale)
    assert np.max(np.abs(got - want)) <= 1e-4


def test_mla_attention_matches_fp64_and_single_position():
    heads, kv_lora, rope, seq = 16, 512, 64, 700
    lat = normal(12, (seq, kv_lora + rope))
    qt, qr = normal(13, (heads, kv_lora)), normal(14, (heads, rope))
    s = 1 / math.sqrt(192)
    assert_close(oracle.mla_attention(lat, qt, qr, kv_lora, rope, s),
                 oracle.mla_attention_f64(lat, qt, qr, kv_lora, rope, s), 1e-5, 1e-5, "mla vs fp64")
    one = oracle.mla_attention(lat[:1], qt, qr, kv_lora, rope, s)
    assert np.array_equal(one, np.tile(lat[0, :kv_lora], (heads, 1)))


# ------------------------------------------------------------------ page accounting
def test_paging_bytes_match_reference_tests():
    """Tests/Program.cs:242-253 (700 tokens -> 3 pages) and :424-438 (300 tokens, 2 layers)."""
    p = paging.IntendedPaging(layers=2, page_bytes=256 * 32 * 4 * 2)
    for pos in range(700):
        p.append(1, pos)
    assert p.seq_len == 700 and p.bytes_used == 3 * 256 * 32 * 4 * 2
    g = paging.IntendedPaging(layers=2, page_bytes=256 * 256 * 4 * 2)
    for pos in range(300):
        for layer in range(2):
            g.append(layer, pos)
    assert g.bytes_used == 2 * 2 * 256 * 256 * 4 * 2


def test_reference_growth_bug_is_where_documented():
    """PagedKvCache.Ensure (:45-57) leaves slot 3 null: sequential Append fails at 768."""
    first, nulls = paging.reference_growth_null_pages(2000)
    assert first == 768 and nulls == [3]
    first, nulls = paging.reference_growth_null_pages(700)
    assert first is None and nulls == [3]


# ------------------------------------------------------------------ weight-row decoders
from tests import quant  # noqa: E402


def test_q4_0_known_answer_from_reference_test():
    """Tests/Program.cs:449-457 (hand-built Q4_0: d = f16(-0.5), bytes 0x08 and 0x2A).  The
    reference's block has 2 more pad bytes (BlockDequantizer.cs:52-69); the nibble order is
    the same: low nibble of byte i is weight i, high nibble weight i+16."""
    blk = np.zeros(20, np.uint8)
    blk[0], blk[1], blk[2], blk[3] = 0x00, 0xB8, 0x08, 0x2A
    y = oracle.dequant_rows(quant.FMT["Q4_0"], blk, 32)[0]
    assert (y[0], y[16], y[1], y[17]) == (0.0, 4.0, -1.0, 3.0)
    assert np.all(y[2:16] == 4.0) and np.all(y[18:] == 4.0)  # zero bytes -> (0-8)*(-0.5)


def test_q8_0_and_fp_rows_closed_form():
    rng = np.random.default_rng(3)
    q = rng.integers(-128, 128, 64).astype(np.int8)
    raw = np.zeros((1, 68), np.uint8)
    for b, d in enumerate((0.25, -3.0)):
        raw[0, 34 * b:34 * b + 2] = np.float16(d).reshape(1).view(np.uint8)
        raw[0, 34 * b + 2:34 * b + 34] = q[32 * b:32 * b + 32].view(np.uint8)
    y = oracle.dequant_rows(quant.FMT["Q8_0"], raw, 64)[0]
    assert np.array_equal(y, np.concatenate([0.25 * q[:32], -3.0 * q[32:]]).astype(F32))
    x = normal(4, (3, 40))
    for name in ("F32", "F16", "BF16"):
        f = quant.FMT[name]
        got = oracle.dequant_rows(f, quant.quantize(f, x), 40)
        want = {"F32": x, "F16": x.astype(np.float16).astype(F32),
                "BF16": oracle.bf16_to_f32(oracle.f32_to_bf16(x))}[name]
        assert np.array_equal(got, want), name


def test_q4_k_layout_closed_form():
    """Every sub-block gets its own 6-bit scale and min (values >= 16 exercise the high-bit
    packing of sub-blocks 4..7) and every nibble a known value; d and dmin are powers of two
    so d*sc*q - dmin*m is exact and the layout alone decides the result."""
    rng = np.random.default_rng(5)
    sc = np.array([1, 7, 16, 63, 33, 17, 48, 5])
    mn = np.array([0, 63, 9, 20, 47, 31, 16, 62])
    q = rng.integers(0, 16, 256)
    d, dmin = 2.0 ** -6, 2.0 ** -9
    blk = quant.build_q4k_block(d, dmin, sc, mn, q)
    assert np.array_equal(blk, quant.pack_q4k(np.array([d]), np.array([dmin]), sc[None], mn[None], q[None])[0])
    y = oracle.dequant_rows(quant.FMT["Q4_K"], blk, 256)[0].astype(np.float64)
    sub = np.arange(256) // 32
    assert np.array_equal(y, d * sc[sub] * q - dmin * mn[sub])


def test_q6_k_layout_closed_form():
    """Each 6-bit value has one low-nibble and one 2-bit slot (the slots tile the 192 bytes
    exactly once) and each group of 16 its own int8 scale."""
    slots = set()
    for w in range(256):
        ql, hi, qh, sh, _ = quant.q6k_slots(w)
        slots.add(("l", ql, hi))
        slots.add(("h", qh, sh))
    assert len(slots) == 512 and {s[1] for s in slots if s[0] == "l"} == set(range(128))
    rng = np.random.default_rng(6)
    q = rng.integers(0, 64, 256)
    sc = np.array([1, -2, 3, -4, 127, -128, 7, 8, 9, -10, 11, 12, -13, 14, 15, 100])
    d = 2.0 ** -10
    blk = quant.build_q6k_block(d, sc, q)
    assert np.array_equal(blk, quant.pack_q6k(np.array([d]), sc[None], q[None])[0])
    y = oracle.dequant_rows(quant.FMT["Q6_K"], blk, 256)[0].astype(np.float64)
    k = np.array([quant.q6k_scale_index(w) for w in range(256)])
    assert np.array_equal(y, d * sc[k] * (q - 32))


@pytest.mark.parametrize("name,tol", [("Q8_0", 0.02), ("Q6_K", 0.03), ("Q4_0", 0.11), ("Q4_K", 0.09)])
def test_quant_round_trip_rms(name, tol):
    """Tests/Program.cs:96-127 (QuantRoundTrip): N(0, 0.5^2) weights, 32 blocks, relative RMS
    within the reference's per-format bound."""
    f = quant.FMT[name]
    bs = quant.BLOCK[f][0]
    x = (np.random.default_rng(7).standard_normal((1, bs * 32)) * 0.5).astype(F32)
    raw = quant.quantize(f, x)
    assert raw.shape[1] == oracle.row_bytes(f, bs * 32)
    y = oracle.dequant_rows(f, raw, bs * 32)
    rms = math.sqrt(np.mean((y - x) ** 2)) / math.sqrt(np.mean(x ** 2))
    assert rms <= tol, f"{name}: rel RMS {rms:.3f}"


def test_row_bytes_and_unsupported_formats():
    assert oracle.row_bytes(quant.FMT["Q4_K"], 512) == 288 and oracle.row_bytes(quant.FMT["Q6_K"], 256) == 210
    assert oracle.row_bytes(quant.FMT["Q4_0"], 64) == 40 and oracle.row_bytes(quant.FMT["F32"], 3) == 12
    for fmt, n in ((5, 256), (8, 64), (quant.FMT["Q8_0"], 48), (quant.FMT["Q4_K"], 128)):
        with pytest.raises(ValueError):
            oracle.row_bytes(fmt, n)


# ------------------------------------------------------------------ fused dequant + dot (DotRow)
@pytest.mark.parametrize("name", ["Q8_0", "Q6_K", "Q4_0", "Q4_K"])
def test_dot_row_matches_dequantized_dot(name):
    """Tests/Program.cs:129-165 (DotMatches): DotRow of each row against the dequantized
    row dotted in fp32, relative error <= 2e-4 (12 rows, 4 blocks each)."""
    f = quant.FMT[name]
    bs = quant.BLOCK[f][0]
    cols, rows = bs * 4, 12
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((rows, cols)) * 0.4).astype(F32)
    x = (rng.standard_normal(cols) * 0.5).astype(F32)
    raw = quant.quantize(f, w)
    wd = oracle.dequant_rows(f, raw, cols)
    y = oracle.matvec(f, raw, cols, x)
    for r in range(rows):
        s = np.float32(0)
        for c in range(cols):
            s = np.float32(s + np.float32(wd[r, c] * x[c]))
        assert abs(y[r] - s) / max(abs(s), 1e-3) <= 2e-4, (name, r, y[r], s)


@pytest.mark.parametrize("name", ["F32", "F16", "BF16"])
def test_dot_row_fp_lane_order(name):
    """SimdMath.DotF32 lane structure: +1e8 and -1e8 in the same lane cancel exactly before
    the +1 of another lane is added (a sequential sum would lose the 1)."""
    f = quant.FMT[name]
    x = np.zeros(16, F32)
    x[0], x[1], x[8] = 1e8, 1.0, -1e8
    w = np.ones((1, 16), F32)
    assert oracle.matvec(f, quant.quantize(f, w), 16, x)[0] == 1.0
    x2 = x.copy()
    x2[9] = -1e8                      # same lane as x[1]: lane 1 = 1 - 1e8 = -1e8
    x2[0] = 1e8
    assert oracle.matvec(f, quant.quantize(f, w), 16, x2)[0] == np.float32(np.float32(1e8 - 1e8) - 1e8 + 0)


def test_dot_row_f16_exponent_31_is_finite():
    """DotKernels.cs:86-100: the vector half converter re-biases exponent 31 like a normal
    exponent (inf 0x7C00 -> 65536, 0x7E00 -> 98304) instead of producing inf/NaN; the scalar
    tail (cols % 8) and the dequantizer keep the exact conversion."""
    w = np.zeros((1, 8), np.uint16)
    w[0, 0], w[0, 3] = 0x7C00, 0x7E00
    x = np.zeros(8, F32)
    x[0], x[3] = 1.0, 2.0
    y = oracle.matvec(quant.FMT["F16"], w.view(np.uint8), 8, x)[0]
    assert y == 65536.0 + 2 * 98304.0
    assert np.isinf(oracle.dequant_rows(quant.FMT["F16"], w.view(np.uint8), 8)[0, 0])


def test_dot_row_q8_0_lane_structure():
    """Q8_0 (DotKernels.cs:183-230): lane L sums q[L], q[8+L], q[16+L], q[24+L]; blocks add in order."""
    raw = np.zeros((1, 34), np.uint8)
    raw[0, 0:2] = np.float16(1.0).reshape(1).view(np.uint8)
    raw[0, 2 + np.array([0, 1, 8])] = 1
    x = np.zeros(32, F32)
    x[0], x[1], x[8] = 1e8, 1.0, -1e8
    assert oracle.matvec(quant.FMT["Q8_0"], raw, 32, x)[0] == 1.0


def test_dot_row_q4_k_order_of_terms():
    """Q4_K (DotKernels.cs:322-358): sum += a*(VecDot16 + VecDot16) - mm*SubSum, sub-blocks in
    order; with one sub-block scale 1 and min 0, the row is a plain lane-structured dot."""
    sc = np.zeros(8, int)
    mn = np.zeros(8, int)
    sc[0] = 1
    q = np.zeros(256, int)
    q[[0, 1, 8]] = 1
    blk = quant.build_q4k_block(1.0, 0.0, sc, mn, q)
    x = np.zeros(256, F32)
    x[0], x[1], x[8] = 1e8, 1.0, -1e8
    assert oracle.matvec(quant.FMT["Q4_K"], blk, 256, x)[0] == 1.0
    mn[1] = 2                       # odd sub-block: -dmin*2*SubSum(x[32:64])
    x[32:64] = 0.5
    blk = quant.build_q4k_block(1.0, 0.25, sc, mn, q)
    assert oracle.matvec(quant.FMT["Q4_K"], blk, 256, x)[0] == np.float32(1.0 - 0.5 * 16.0)
