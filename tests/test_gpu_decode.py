"""GPU parity of the paged-KV GQA path (PagedKvCache.cs:41-136) through the C ABI.

Tolerances (fp32 accumulation on exactly decoded KV): max-abs <= 1e-3 and
relative L2 <= 1e-4 against the oracle's op-order restatement of the
reference; each case also reports the error of both sides against fp64.
"""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.util import assert_close, errors, normal, to_dtype_bits

pytestmark = pytest.mark.gpu

TOL_ABS, TOL_REL = 1e-3, 1e-4


def oracle_decode(K, V, q, heads, kv_heads, D, scale):
    return oracle.kv_attention(K, V, q, heads, kv_heads, D, scale)


def check_decode(got, K, V, q, heads, kv_heads, D, scale, what):
    want = oracle_decode(K, V, q, heads, kv_heads, D, scale)
    a, r = assert_close(got, want, TOL_ABS, TOL_REL, what)
    f64 = oracle.kv_attention_f64(K, V, q, heads, kv_heads, D, scale)
    ga, gr = errors(got, f64)
    oa, orr = errors(want, f64)
    print(f"{what}: vs oracle max-abs {a:.2e} rel {r:.2e} | vs fp64: gpu {gr:.2e} oracle {orr:.2e}")


# ------------------------------------------------------------------ the reference's own tests
@pytest.mark.parametrize("heads,kv_heads,tokens,layers,layer", [(4, 2, 700, 2, 1), (2, 2, 600, 1, 0)])
def test_reference_kvcache_invariants(gpu, heads, kv_heads, tokens, layers, layer):
    """Tests/Program.cs:242-280 and Cli/Commands.cs:3037-3065, appended one row at a time."""
    D = 16
    kv_dim = kv_heads * D
    i = np.arange(kv_dim)
    k, v = np.sin(i).astype(np.float32), np.cos(i).astype(np.float32)
    with qr.PagedKvCache(layers, heads, kv_heads, D, 1000) as kv:
        for pos in range(tokens):
            kv.Append(layer, pos, k, v)
        assert kv.SeqLen == tokens
        assert kv.BytesUsed == 3 * 256 * kv_dim * 4 * 2
        for qv in (0.0, 1.0):
            out = kv.Attention(layer, tokens - 1, np.full(heads * D, qv, np.float32), 0.25)
            for h in range(heads):
                kvh = h * kv_heads // heads
                assert np.max(np.abs(out[h * D:(h + 1) * D] - v[kvh * D:(kvh + 1) * D])) <= 1e-4


def test_sequential_append_past_page_growth_bug(gpu):
    """Sequential Append at 768+ works (the reference's Ensure leaves page 3 null there)."""
    heads, kv_heads, D, n = 8, 2, 64, 1100
    K, V = normal(40, (n, kv_heads * D)), normal(41, (n, kv_heads * D))
    q = normal(42, heads * D)
    with qr.PagedKvCache(1, heads, kv_heads, D, 2048) as kv:
        for pos in range(n):
            kv.Append(0, pos, K[pos], V[pos])
        assert kv.BytesUsed == 5 * 256 * kv_heads * D * 4 * 2
        for pos in (767, 768, 1023, n - 1):
            check_decode(kv.Attention(0, pos, q, 0.125), K[:pos + 1], V[:pos + 1], q, heads, kv_heads, D,
                         0.125, f"seq append pos {pos}")


# ------------------------------------------------------------------ configuration 1 and shapes
def test_c1_tiny_gqa_fp32(gpu):
    """8 query heads, 2 kv heads, head_dim 64, 512 cached tokens (2 pages), scale 1/8."""
    heads, kv_heads, D, seq = 8, 2, 64, 512
    q = normal(100, heads * D)
    K, V = normal(101, (seq, kv_heads * D)), normal(102, (seq, kv_heads * D))
    with qr.PagedKvCache(1, heads, kv_heads, D, seq) as kv:
        kv.AppendRange(0, 0, K, V)
        check_decode(kv.Attention(0, seq - 1, q, 0.125), K, V, q, heads, kv_heads, D, 0.125, "C1")


@pytest.mark.parametrize("heads,kv_heads,D,seq", [
    (6, 4, 16, 300),     # uneven GQA map, one query head per workgroup
    (5, 3, 32, 777),
    (16, 2, 256, 400),   # G = 8, head_dim 256
    (64, 8, 128, 1300),  # G = 8
    (32, 2, 128, 600),   # G = 16: two head chunks per kv head
    (1, 1, 64, 1),       # single position
    (12, 4, 64, 2049),   # G = 3
    (14, 2, 128, 257),   # G = 7
])
def test_decode_shapes(gpu, heads, kv_heads, D, seq):
    q = normal(seq, heads * D)
    K, V = normal(seq + 1, (seq, kv_heads * D)), normal(seq + 2, (seq, kv_heads * D))
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, seq + 5) as kv:
        kv.AppendRange(0, 0, K, V)
        check_decode(kv.Attention(0, seq - 1, q, scale), K, V, q, heads, kv_heads, D, scale,
                     f"H{heads}/Hkv{kv_heads}/D{D}/seq{seq}")
        if seq > 3:  # a shorter query over the same pages
            p = seq // 3
            check_decode(kv.Attention(0, p, q, scale), K[:p + 1], V[:p + 1], q, heads, kv_heads, D, scale,
                         f"H{heads}/Hkv{kv_heads}/D{D}/pos{p}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D,seq", [
    (64, 8, 128, 1300),  # G = 8 (70B shape)
    (32, 2, 128, 600),   # G = 16: one full MFMA column block
    (48, 2, 128, 900),   # G = 24: two head chunks (16 + 8)
    (12, 4, 64, 2049),   # G = 3, head_dim 64
    (14, 2, 128, 257),   # G = 7, one position into the second page
    (6, 4, 64, 300),     # uneven GQA map, one query head per workgroup
    (1, 1, 64, 1),       # single position
])
def test_decode_16bit_mfma_shapes(gpu, dtype, heads, kv_heads, D, seq):
    """16-bit caches with head_dim 64/128 decode on MFMA tiles (pages in the MFMA operand layout)
    with hi/lo-split q and P: still the fp32-accumulation tolerance."""
    q = normal(seq + 7, heads * D)
    Kb, K = to_dtype_bits(normal(seq + 8, (seq, kv_heads * D)), dtype)
    Vb, V = to_dtype_bits(normal(seq + 9, (seq, kv_heads * D)), dtype)
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, seq + 5, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        kr, vr = kv.Read(0, 0, seq)
        assert np.array_equal(kr, Kb) and np.array_equal(vr, Vb)  # layout round trip
        check_decode(kv.Attention(0, seq - 1, q, scale), K, V, q, heads, kv_heads, D, scale,
                     f"{dtype} H{heads}/Hkv{kv_heads}/D{D}/seq{seq}")
        if seq > 3:
            p = seq // 3
            check_decode(kv.Attention(0, p, q, scale), K[:p + 1], V[:p + 1], q, heads, kv_heads, D, scale,
                         f"{dtype} H{heads}/Hkv{kv_heads}/D{D}/pos{p}")


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("heads,kv_heads,D,seq", [
    (32, 8, 80, 1500),   # 10 chunks of 8 per row, rounded up to 16 lanes
    (16, 4, 96, 2049),
    (8, 2, 120, 700),
    (12, 4, 40, 513),
    (4, 1, 200, 300),    # 25 chunks, rounded up to 32 lanes
    (6, 3, 24, 777),
    (5, 5, 136, 256),    # one query head per kv head, exactly one page
])
def test_decode_head_dims_not_a_power_of_two(gpu, dtype, heads, kv_heads, D, seq):
    """PagedKvCache takes any headDim (PagedKvCache.cs:29-37); multiples of 8 that are not
    powers of two run on the streaming kernel with the row's last lanes masked.  Rows past
    the attended position hold NaN, so a masked lane that read a neighbour would show."""
    q = normal(seq + 40, heads * D)
    Kb, K = to_dtype_bits(normal(seq + 41, (seq, kv_heads * D)), dtype)
    Vb, V = to_dtype_bits(normal(seq + 42, (seq, kv_heads * D)), dtype)
    if dtype == "f32":
        nanb = np.full((64, kv_heads * D), np.nan, np.float32)
    else:  # quiet NaN bit patterns
        nanb = np.full((64, kv_heads * D), 0x7E00 if dtype == "f16" else 0x7FC0, np.uint16)
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, seq + 64, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        kv.AppendRange(0, seq, nanb, nanb, src_dtype=dtype)
        kr, vr = kv.Read(0, 0, seq)
        assert np.array_equal(kr, Kb) and np.array_equal(vr, Vb)
        check_decode(kv.Attention(0, seq - 1, q, scale), K, V, q, heads, kv_heads, D, scale,
                     f"{dtype} H{heads}/Hkv{kv_heads}/D{D}/seq{seq}")
        p = seq // 3
        check_decode(kv.Attention(0, p, q, scale), K[:p + 1], V[:p + 1], q, heads, kv_heads, D, scale,
                     f"{dtype} H{heads}/Hkv{kv_heads}/D{D}/pos{p}")
        if dtype != "f32":  # causal queries over the same pages (the per-query fallback path)
            qs = normal(seq + 43, (3, heads * D))
            out = kv.AttentionChunk(0, seq - 3, qs, scale)
            for i in range(3):
                check_decode(out[i], K[:seq - 2 + i], V[:seq - 2 + i], qs[i], heads, kv_heads, D, scale,
                             f"{dtype} D{D} chunk query {i}")


@pytest.mark.parametrize("dtype,D", [("f32", 128), ("f16", 128), ("bf16", 64), ("f16", 32)])
def test_stale_nan_rows_past_the_position_are_ignored(gpu, dtype, D):
    """Rows past the attended position that still hold NaN (an earlier sequence,
    then Truncate) never reach the result: the reference reads rows 0..pos only."""
    heads, kv_heads, n, pos = 8, 2, 600, 300
    K, V = normal(120, (n, kv_heads * D)), normal(121, (n, kv_heads * D))
    Kb, Kd = to_dtype_bits(K, dtype)
    Vb, Vd = to_dtype_bits(V, dtype)
    nanb = np.full_like(Kb, np.nan) if dtype == "f32" else np.full_like(Kb, 0x7E00 if dtype == "f16" else 0x7FC0)
    q = normal(122, heads * D)
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, nanb, nanb, src_dtype=dtype)
        kv.Truncate(0)
        kv.AppendRange(0, 0, Kb[:pos + 1], Vb[:pos + 1], src_dtype=dtype)
        got = kv.Attention(0, pos, q, scale)
        assert np.isfinite(got).all()
        check_decode(got, Kd[:pos + 1], Vd[:pos + 1], q, heads, kv_heads, D, scale, f"stale NaN {dtype} D{D}")
        if D in (64, 128) and dtype != "f32":  # chunk path: queries pos-3..pos over the same pages
            qs = normal(123, (4, heads * D))
            out = kv.AttentionChunk(0, pos - 3, qs, scale)
            assert np.isfinite(out).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_16bit_append_bits_and_decode(gpu, dtype):
    """fp32 rows appended into a 16-bit cache take the reference codec's bits
    (FloatToF16 / FloatToBf16); attention then runs on the exactly decoded values."""
    heads, kv_heads, D, seq = 8, 2, 128, 700
    K, V = normal(50, (seq, kv_heads * D)) * 3, normal(51, (seq, kv_heads * D))
    K[0, :4] = [1 + 2 ** -11, -(1 + 2 ** -11), 70000.0, 2 ** -25]  # ties, overflow, subnormal
    q = normal(52, heads * D)
    enc = oracle.f32_to_f16 if dtype == "f16" else oracle.f32_to_bf16
    dec = oracle.f16_to_f32 if dtype == "f16" else oracle.bf16_to_f32
    with qr.PagedKvCache(1, heads, kv_heads, D, seq, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, K[:300], V[:300])
        for pos in range(300, seq):
            kv.Append(0, pos, K[pos], V[pos])
        kb, vb = kv.Read(0, 0, seq)
        assert np.array_equal(kb, enc(K)) and np.array_equal(vb, enc(V))
        Kd, Vd = dec(kb), dec(vb)
        Kd[0, 2] = 0.0  # keep the inf out of the score check below
        kv.AppendRange(0, 0, enc(Kd[:1]), enc(Vd[:1]), src_dtype=dtype)
        kb2, _ = kv.Read(0, 0, 1)
        assert np.array_equal(kb2, enc(Kd[:1]))
        check_decode(kv.Attention(0, seq - 1, q, 1 / math.sqrt(D)), Kd, Vd, q, heads, kv_heads, D,
                     1 / math.sqrt(D), f"{dtype} cache")


def test_batch_independent_page_tables(gpu):
    """Four sequences appended interleaved, so their pages alternate in the pool."""
    heads, kv_heads, D = 32, 8, 128
    lens = [1000, 257, 1, 780]
    data = [(normal(60 + s, (n, kv_heads * D)), normal(70 + s, (n, kv_heads * D))) for s, n in enumerate(lens)]
    with qr.PagedKvCache(2, heads, kv_heads, D, 1024, max_batch=4) as kv:
        step = 128
        for p0 in range(0, max(lens), step):
            for s, n in enumerate(lens):
                if p0 < n:
                    e = min(n, p0 + step)
                    kv.AppendRange(1, p0, data[s][0][p0:e], data[s][1][p0:e], seq_id=s)
        for s, n in enumerate(lens):
            assert kv.seq_len(s) == n
        q = normal(80, (4, heads * D))
        out = kv.AttentionBatch(1, [0, 1, 2, 3], [n - 1 for n in lens], q, 0.088)
        for s, n in enumerate(lens):
            check_decode(out[s], data[s][0], data[s][1], q[s], heads, kv_heads, D, 0.088, f"batch seq {s}")
        # the same entry twice and out of order
        out2 = kv.AttentionBatch(1, [3, 0, 3], [lens[3] - 1, lens[0] - 1, 100], q[[3, 0, 1]], 0.088)
        assert_close(out2[0], out[3], 1e-6, 1e-5, "repeat entry 3")
        assert_close(out2[1], out[0], 1e-6, 1e-5, "repeat entry 0")
        check_decode(out2[2], data[3][0][:101], data[3][1][:101], q[1], heads, kv_heads, D, 0.088, "batch pos 100")


@pytest.mark.parametrize("q_dtype", ["f32", "f16", "bf16"])
def test_chunk_causal_matches_sequential_calls(gpu, q_dtype):
    """Query i at pos0+i sees 0..pos0+i: nq sequential Attention calls (SpeculativeRunner.cs:85-93)."""
    heads, kv_heads, D, pos0, nq = 16, 4, 64, 1500, 70
    n = pos0 + nq
    K, V = normal(90, (n, kv_heads * D)), normal(91, (n, kv_heads * D))
    qbits, qf = to_dtype_bits(normal(92, (nq, heads * D)), q_dtype)
    with qr.PagedKvCache(1, heads, kv_heads, D, 4096) as kv:
        kv.AppendRange(0, 0, K, V)
        out = kv.AttentionChunk(0, pos0, qbits, 0.125, q_dtype=q_dtype)
        for i in (0, 1, 33, nq - 1):
            check_decode(out[i], K[:pos0 + i + 1], V[:pos0 + i + 1], qf[i], heads, kv_heads, D, 0.125,
                         f"chunk {q_dtype} query {i}")
        single = kv.Attention(0, pos0 + 5, qf[5], 0.125)
        np.testing.assert_allclose(out[5], single, rtol=0, atol=1e-6)


# ------------------------------------------------------------------ state and errors
def test_truncate_reset_and_overwrite(gpu):
    heads, kv_heads, D = 4, 2, 32
    K, V = normal(110, (600, kv_heads * D)), normal(111, (600, kv_heads * D))
    K2, V2 = normal(112, (600, kv_heads * D)), normal(113, (600, kv_heads * D))
    q = normal(114, heads * D)
    with qr.PagedKvCache(1, heads, kv_heads, D, 1000) as kv:
        kv.AppendRange(0, 0, K, V)
        used = kv.BytesUsed
        kv.Truncate(1000)
        assert kv.SeqLen == 600
        kv.Truncate(300)                      # PagedKvCache.cs:76: O(1), pages kept
        assert kv.SeqLen == 300 and kv.BytesUsed == used
        kv.AppendRange(0, 300, K2[300:400], V2[300:400])  # rewrite after rollback
        assert kv.SeqLen == 400
        Km = np.concatenate([K[:300], K2[300:400]])
        Vm = np.concatenate([V[:300], V2[300:400]])
        check_decode(kv.Attention(0, 399, q, 0.2), Km, Vm, q, heads, kv_heads, D, 0.2, "after truncate")
        kv.Reset()
        assert kv.SeqLen == 0 and kv.BytesUsed == used  # PagedKvCache.cs:72: pages reused
        kv.Append(0, 0, K2[0], V2[0])
        assert kv.SeqLen == 1
        assert np.array_equal(kv.Attention(0, 0, q, 0.2)[:D], V2[0, :D])  # one position: exact V row


def test_error_paths(gpu):
    heads, kv_heads, D = 4, 2, 16
    with qr.PagedKvCache(2, heads, kv_heads, D, 600) as kv:
        row = np.ones(kv_heads * D, np.float32)
        with pytest.raises(qr.QrOutOfRange):
            kv.Append(0, 600, row, row)                 # pos >= max_seq
        with pytest.raises(qr.QrOutOfRange):
            kv.Append(0, 0, np.ones(kv_heads * D + 1, np.float32), row)  # longer than kv_dim
        with pytest.raises(qr.QrInvalidArgument):
            kv.Append(2, 0, row, row)                   # layer out of range
        with pytest.raises(qr.QrNotResident):
            kv.Attention(0, 10, np.zeros(heads * D, np.float32), 1.0)  # nothing appended
        kv.Append(0, 0, row, row)
        kv.Attention(0, 255, np.zeros(heads * D, np.float32), 1.0)      # page 0 resident
        with pytest.raises(qr.QrNotResident):
            kv.Attention(0, 256, np.zeros(heads * D, np.float32), 1.0)
        with pytest.raises(qr.QrNotResident):
            kv.Attention(1, 0, np.zeros(heads * D, np.float32), 1.0)   # other layer
        with pytest.raises(qr.QrInvalidArgument):
            kv.AttentionBatch(0, [1], [0], np.zeros(heads * D, np.float32), 1.0)  # seq_id >= max_batch
        # a short row overwrites only its prefix (Span.CopyTo semantics)
        kv.Append(0, 1, np.full(kv_heads * D, 2, np.float32), np.full(kv_heads * D, 3, np.float32))
        kv.Append(0, 1, np.full(5, 7, np.float32), np.full(0, 0, np.float32))
        k1, v1 = kv.Read(0, 1, 1)
        assert np.array_equal(k1[0], np.r_[np.full(5, 7), np.full(kv_heads * D - 5, 2)].astype(np.float32))
        assert np.all(v1 == 3)
        assert kv.BytesPerToken == kv_heads * D * 4 * 2 * 2


# ------------------------------------------------------------------ full-size configurations
def rope_inputs(heads, kv_heads, D, n, seed, theta=500000.0):
    """Q (at position n-1) and K rows with RoPE at their positions; V plain."""
    q = oracle.rope_rows(normal(seed, (1, heads * D)), D, n - 1, theta).reshape(-1)
    K = oracle.rope_rows(normal(seed + 1, (n, kv_heads * D)), D, 0, theta)
    V = normal(seed + 2, (n, kv_heads * D))
    return q, K, V


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_c2_llama8b_decode_32k(gpu, dtype):
    """32 query heads, 8 kv heads, head_dim 128, 32,768 cached tokens (128 pages), RoPE 5e5."""
    heads, kv_heads, D, n = 32, 8, 128, 32768
    q, K, V = rope_inputs(heads, kv_heads, D, n, 200)
    Kb, Kd = to_dtype_bits(K, dtype)
    Vb, Vd = to_dtype_bits(V, dtype)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        assert kv.BytesUsed == 128 * 256 * kv_heads * D * (4 if dtype == "f32" else 2) * 2
        check_decode(kv.Attention(0, n - 1, q, 1 / math.sqrt(D)), Kd, Vd, q, heads, kv_heads, D,
                     1 / math.sqrt(D), f"C2 {dtype} B1")


def test_c2_llama8b_decode_32k_batch16_fp16(gpu):
    """Batch 16 with independent page tables (sequences appended round-robin by page); every
    sequence's Q and K carry RoPE at base 500000 (Q at position 32,767), as at batch 1."""
    heads, kv_heads, D, n, B = 32, 8, 128, 32768, 16
    seqs = []
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="f16", max_batch=B) as kv:
        kv.Reserve(B * 128)
        qs = []
        for b in range(B):
            q, K, V = rope_inputs(heads, kv_heads, D, n, 300 + 3 * b)
            seqs.append((K.astype(np.float16), V.astype(np.float16)))
            qs.append(q)
        for p0 in range(0, n, 4096):  # interleave so page tables are not contiguous runs
            for b in range(B):
                kv.AppendRange(0, p0, seqs[b][0][p0:p0 + 4096].view(np.uint16),
                               seqs[b][1][p0:p0 + 4096].view(np.uint16), src_dtype="f16", seq_id=b)
        q = np.stack(qs)
        pos = [n - 1] * B
        out = kv.AttentionBatch(0, list(range(B)), pos, q, 1 / math.sqrt(D))
        for b in (0, 9, 15):
            K, V = seqs[b]
            check_decode(out[b], K.astype(np.float32), V.astype(np.float32), q[b], heads, kv_heads, D,
                         1 / math.sqrt(D), f"C2 f16 B16 entry {b}")
        for b in (3, 12):  # a batched entry equals the same query alone (split sizes follow the batch)
            assert_close(kv.Attention(0, n - 1, q[b], 1 / math.sqrt(D), seq_id=b), out[b], 1e-6, 1e-5,
                         f"B16 entry {b} vs single")


def test_c4_llama70b_decode_128k_fp16(gpu):
    """64 query heads, 8 kv heads, head_dim 128, 131,072 cached fp16 tokens (512 pages)."""
    heads, kv_heads, D, n = 64, 8, 128, 131072
    rng = np.random.default_rng(500)
    K = rng.standard_normal((n, kv_heads * D), dtype=np.float32).astype(np.float16)
    V = rng.standard_normal((n, kv_heads * D), dtype=np.float32).astype(np.float16)
    q = normal(501, heads * D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n + 8, kv_dtype="f16") as kv:
        kv.AppendRange(0, 0, K.view(np.uint16), V.view(np.uint16), src_dtype="f16")
        got = kv.Attention(0, n - 1, q, 1 / math.sqrt(D))
    check_decode(got, K.astype(np.float32), V.astype(np.float32), q, heads, kv_heads, D, 1 / math.sqrt(D),
                 "C4 decode f16")


def test_c2_llama8b_decode_32k_batch16_fp32(gpu):
    """Batch 16 of 32,768 fp32 tokens each, pages of the 16 sequences interleaved in the pool,
    Q and K with RoPE at base 500000 (Q at position 32,767).  This batch takes the plan of 16
    pages per split (8 splits per entry), the longest split plan of the streaming kernel;
    single-sequence calls take 4 pages per split."""
    import torch

    heads, kv_heads, D, n, B = 32, 8, 128, 32768, 16
    kv_dim, chunk, scale, theta = kv_heads * D, 4096, 1 / math.sqrt(D), 500000.0
    checked = (0, 7, 15)
    host = {b: ([], []) for b in checked}
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="f32", max_batch=B) as kv:
        kv.Reserve(B * 128)
        for p0 in range(0, n, chunk):  # interleave so page tables are not contiguous runs
            for b in range(B):
                seed = 600 + 1000 * b + 2 * (p0 // chunk)
                K = oracle.rope_rows(normal(seed, (chunk, kv_dim)), D, p0, theta)
                V = normal(seed + 1, (chunk, kv_dim))
                kv.AppendRangeDev(0, p0, torch.from_numpy(K).to(gpu), torch.from_numpy(V).to(gpu), seq_id=b)
                if b in host:
                    host[b][0].append(K)
                    host[b][1].append(V)
        torch.cuda.synchronize()
        assert kv.BytesUsed == B * 128 * 256 * kv_dim * 4 * 2
        ids, pos = list(range(B)), [n - 1] * B
        assert kv.DecodePlan(0, ids, pos) == (16 * 256, 8)
        q = np.stack([oracle.rope_rows(normal(601 + b, (1, heads * D)), D, n - 1, theta).reshape(-1)
                      for b in range(B)])
        out = kv.AttentionBatch(0, ids, pos, q, scale)
        for b in checked:
            K, V = np.concatenate(host[b][0]), np.concatenate(host[b][1])
            check_decode(out[b], K, V, q[b], heads, kv_heads, D, scale, f"C2 f32 B16 entry {b}")
        assert kv.DecodePlan(0, [7], [n - 1]) == (4 * 256, 32)
        assert_close(kv.Attention(0, n - 1, q[7], scale, seq_id=7), out[7], 1e-6, 1e-5, "B16 entry 7 vs single")
        # the device entry point gives the batch call's result
        qd = torch.from_numpy(q).to(gpu)
        od = torch.empty_like(qd)
        kv.AttentionDev(0, ids, pos, qd, od, scale)
        torch.cuda.synchronize()
        assert np.array_equal(od.cpu().numpy(), out)


@pytest.mark.parametrize("D,heads,kv_heads", [(16, 64, 32), (32, 32, 32)])
def test_decode_fp32_sixteen_page_splits(gpu, D, heads, kv_heads):
    """Small kv rows and a batch large enough that the plan takes 16 pages per split, with a
    ragged last split (one entry ends inside a page, one spans fewer pages than a split)."""
    lens = [10240, 9000, 5000, 10240]
    B, kv_dim, scale = len(lens), kv_heads * D, 1 / math.sqrt(D)
    data = [(normal(700 + 2 * b, (n, kv_dim)), normal(701 + 2 * b, (n, kv_dim))) for b, n in enumerate(lens)]
    with qr.PagedKvCache(1, heads, kv_heads, D, max(lens), max_batch=B) as kv:
        for p0 in range(0, max(lens), 2048):
            for b, n in enumerate(lens):
                if p0 < n:
                    e = min(n, p0 + 2048)
                    kv.AppendRange(0, p0, data[b][0][p0:e], data[b][1][p0:e], seq_id=b)
        ids, pos = list(range(B)), [n - 1 for n in lens]
        assert kv.DecodePlan(0, ids, pos) == (16 * 256, 3)
        q = normal(710, (B, heads * D))
        out = kv.AttentionBatch(0, ids, pos, q, scale)
        for b, n in enumerate(lens):
            check_decode(out[b], data[b][0], data[b][1], q[b], heads, kv_heads, D, scale,
                         f"16-page splits D{D} entry {b} ({n} tokens)")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_split_merge_over_many_back_to_back_calls(gpu, dtype):
    """Split partials of many calls queued back to back on one handle (alternating layers and
    batch sizes, new queries each time, no host synchronisation between them): each call
    must match the oracle, so a partial left over from an earlier call, or merged into the
    wrong entry, shows up as a mismatch."""
    import torch

    heads, kv_heads, D, n = 32, 8, 128, 8192
    scale = 1 / math.sqrt(D)
    data = []
    with qr.PagedKvCache(2, heads, kv_heads, D, n, kv_dtype=dtype, max_batch=3) as kv:
        for layer in range(2):
            for s in range(3):
                Kb, Kd = to_dtype_bits(normal(800 + 10 * layer + s, (n, kv_heads * D)), dtype)
                Vb, Vd = to_dtype_bits(normal(850 + 10 * layer + s, (n, kv_heads * D)), dtype)
                kv.AppendRange(layer, 0, Kb, Vb, src_dtype=dtype, seq_id=s)
                data.append((Kd, Vd))
        calls = []
        for i in range(48):
            layer, nb = i % 2, 1 + i % 3
            pos = [n - 1 - 37 * ((i + s) % 5) for s in range(nb)]
            q = torch.from_numpy(normal(900 + i, (nb, heads * D))).to(gpu)
            out = torch.empty_like(q)
            kv.AttentionDev(layer, list(range(nb)), pos, q, out, scale)
            calls.append((layer, pos, q, out))
        torch.cuda.synchronize()
        for i, (layer, pos, q, out) in enumerate(calls):
            got, qh = out.cpu().numpy(), q.cpu().numpy()
            for s, p in enumerate(pos):
                if (i + s) % 4:  # a sample of the entries against the oracle
                    continue
                K, V = data[3 * layer + s]
                assert_close(got[s], oracle_decode(K[:p + 1], V[:p + 1], qh[s], heads, kv_heads, D, scale),
                             TOL_ABS, TOL_REL, f"{dtype} call {i} entry {s}")
