"""Seeded random sweep of the decode, chunk and MLA paths against the oracle: shapes drawn
across the spaces the named configurations sample only at points (group sizes with and
without kv_heads dividing heads, head_dim 16..256 including 80 and 96, fp32 and 16-bit
caches, 16-bit and fp32 queries, sequence lengths from 1 to a few thousand, ragged
batches, chunk positions from 0).

Reference semantics: PagedKvCache.Attention (PagedKvCache.cs:83-136) per entry; a chunk
query i at pos0 + i equals that call at its own position (StreamingEngine.cs:831-836); the
MLA absorbed attention of MlaLayer (StreamingEngine.cs:531-568) over the latent cache.
Tolerances are the repository's: decode max-abs <= 1e-3 and rel-L2 <= 1e-4 (fp32
accumulation on exactly decoded KV, q and P as hi + lo parts on the MFMA path); chunk
rel-L2 <= 5e-3 (bf16 caches), 1e-3 (fp16), 1e-4 (fp32); MLA rel-L2 <= 5e-3 (16-bit
latents on MFMA tiles) and 1e-4 (fp32 latents), max-abs <= 1e-3.
"""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.util import assert_close, to_dtype_bits

pytestmark = pytest.mark.gpu

SEED = 20261202
HEAD_DIMS = [16, 32, 64, 80, 96, 128, 256]


def _decode_cases(n=24):
    rng = np.random.default_rng(SEED)
    out = []
    for i in range(n):
        kv_heads = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 8, 16]))
        heads = kv_heads * g + (1 if i % 6 == 5 and kv_heads > 1 else 0)  # kv_heads not dividing heads
        D = int(rng.choice(HEAD_DIMS))
        dtype = str(rng.choice(["f32", "f16", "bf16"]))
        batch = int(rng.integers(1, 4))
        seqs = [int(rng.integers(1, 3000)) for _ in range(batch)]
        out.append((i, heads, kv_heads, D, dtype, tuple(seqs)))
    return out


def _chunk_cases(n=10):
    rng = np.random.default_rng(SEED + 1)
    out = []
    for i in range(n):
        kv_heads = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 8]))
        dtype = str(rng.choice(["f32", "f16", "bf16"]))
        D = int(rng.choice([64, 128])) if dtype != "f32" else int(rng.choice([32, 64, 80, 128]))
        q_dtype = str(rng.choice(["f32", "f16", "bf16"]))
        nq = int(rng.integers(1, 80))
        pos0 = int(rng.integers(0, 2500))
        out.append((i, kv_heads * g, kv_heads, D, dtype, q_dtype, nq, pos0))
    return out


@pytest.mark.parametrize("case", _decode_cases(), ids=lambda c: "d{}-H{}-K{}-D{}-{}-{}".format(*c[:5], "x".join(map(str, c[5]))))
def test_decode_sweep(gpu, case):
    i, heads, kv_heads, D, dtype, seqs = case
    rng = np.random.default_rng(SEED + 100 + i)
    kv_dim = kv_heads * D
    scale = 1 / math.sqrt(D)
    n = max(seqs)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype=dtype, max_batch=len(seqs)) as kv:
        data = []
        for b, s in enumerate(seqs):
            Kb, Kd = to_dtype_bits(rng.standard_normal((s, kv_dim), dtype=np.float32), dtype)
            Vb, Vd = to_dtype_bits(rng.standard_normal((s, kv_dim), dtype=np.float32), dtype)
            kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype, seq_id=b)
            data.append((Kd, Vd))
        q = rng.standard_normal((len(seqs), heads * D), dtype=np.float32)
        out = kv.AttentionBatch(0, list(range(len(seqs))), [s - 1 for s in seqs], q, scale)
    for b, (Kd, Vd) in enumerate(data):
        want = oracle.kv_attention(Kd, Vd, q[b], heads, kv_heads, D, scale)
        assert_close(out[b], want, 1e-3, 1e-4, f"decode sweep case {i} entry {b} (seq {seqs[b]})")


@pytest.mark.parametrize("case", _chunk_cases(), ids=lambda c: "c{}-H{}-K{}-D{}-{}-q{}-n{}-p{}".format(*c))
def test_chunk_sweep(gpu, case):
    i, heads, kv_heads, D, dtype, q_dtype, nq, pos0 = case
    rng = np.random.default_rng(SEED + 200 + i)
    kv_dim = kv_heads * D
    scale = 1 / math.sqrt(D)
    n = pos0 + nq
    Kb, Kd = to_dtype_bits(rng.standard_normal((n, kv_dim), dtype=np.float32), dtype)
    Vb, Vd = to_dtype_bits(rng.standard_normal((n, kv_dim), dtype=np.float32), dtype)
    qb, qd = to_dtype_bits(rng.standard_normal((nq, heads * D), dtype=np.float32), q_dtype)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        out = kv.AttentionChunk(0, pos0, qb, scale, q_dtype=q_dtype)
    tol = {"bf16": 5e-3, "f16": 1e-3, "f32": 1e-4}[dtype]
    for j in sorted({0, nq // 2, nq - 1}):
        want = oracle.kv_attention(Kd[:pos0 + j + 1], Vd[:pos0 + j + 1], qd[j], heads, kv_heads, D, scale)
        assert_close(out[j], want, 1e-3, tol, f"chunk sweep case {i} query {j} (pos {pos0 + j})")


def _mla_cases(n=10):
    rng = np.random.default_rng(SEED + 2)
    out = []
    for i in range(n):
        dtype = str(rng.choice(["f32", "f16", "bf16"]))
        kv_lora = 512 if dtype != "f32" or i % 2 else int(rng.choice([64, 96, 512]))
        rope = int(rng.choice([0, 64]))
        heads = int(rng.integers(1, 129))
        seq = int(rng.integers(1, 6000))
        pos = int(rng.integers(0, seq))
        out.append((i, dtype, heads, kv_lora, rope, seq, pos))
    return out


@pytest.mark.parametrize("case", _mla_cases(), ids=lambda c: "m{}-{}-H{}-L{}-R{}-n{}-p{}".format(*c))
def test_mla_sweep(gpu, case):
    i, dtype, heads, kv_lora, rope, seq, pos = case
    rng = np.random.default_rng(SEED + 300 + i)
    bits, latd = to_dtype_bits(rng.standard_normal((seq, kv_lora + rope), dtype=np.float32), dtype)
    qt = rng.standard_normal((heads, kv_lora), dtype=np.float32)
    qrp = rng.standard_normal((heads, rope), dtype=np.float32)
    scale = 1 / math.sqrt(192)
    with qr.MlaLatentCache(1, kv_lora + rope, seq, dtype=dtype, rope=rope) as m:
        m.AppendRange(0, 0, bits, src_dtype=dtype)
        got = m.AbsorbedAttention(0, pos, qt, qrp, scale)
    want = oracle.mla_attention(latd[:pos + 1], qt, qrp, kv_lora, rope, scale)
    assert_close(got, want, 1e-3, 1e-4 if dtype == "f32" else 5e-3, f"MLA sweep case {i} (pos {pos})")
