"""GPU parity of causal multi-query attention (chunked prefill, speculative verify).

Reference semantics: query i at position pos0+i equals a PagedKvCache.Attention
call at that position over rows 0..pos0+i (StreamingEngine.cs:831-836,
SpeculativeRunner.cs:85-93); the oracle is run on the exactly decoded 16-bit values.
16-bit caches run on MFMA tiles in the cache's own type (queries of another type as
hi + lo parts, P rounded to the cache type): tolerance max-abs <= 1e-3 and rel-L2
<= 5e-3 for bf16 caches, <= 1e-3 for fp16 caches.  Both sides' errors against fp64
are printed.
"""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.util import assert_close, errors, to_dtype_bits

pytestmark = pytest.mark.gpu

TOL_REL = {"bf16": 5e-3, "f16": 1e-3}


def make(seed, n, kv_dim, dtype):
    rng = np.random.default_rng(seed)
    K = rng.standard_normal((n, kv_dim), dtype=np.float32)
    V = rng.standard_normal((n, kv_dim), dtype=np.float32)
    Kb, Kd = to_dtype_bits(K, dtype)
    Vb, Vd = to_dtype_bits(V, dtype)
    return Kb, Kd, Vb, Vd


def check_query(out_i, Kd, Vd, q_i, heads, kv_heads, D, scale, tol_rel, what):
    want = oracle.kv_attention(Kd, Vd, q_i, heads, kv_heads, D, scale)
    a, r = assert_close(out_i, want, 1e-3, tol_rel, what)
    f64 = oracle.kv_attention_f64(Kd, Vd, q_i, heads, kv_heads, D, scale)
    print(f"{what}: vs oracle max-abs {a:.2e} rel {r:.2e} | vs fp64 gpu {errors(out_i, f64)[1]:.2e} "
          f"oracle {errors(want, f64)[1]:.2e}")


def test_c3_chunked_prefill_bf16(gpu):
    """32 q heads / 8 kv heads / head_dim 128: 2048 bf16 queries after 6144 cached tokens."""
    heads, kv_heads, D, pos0, nq = 32, 8, 128, 6144, 2048
    n = pos0 + nq
    Kb, Kd, Vb, Vd = make(600, n, kv_heads * D, "bf16")
    qb, qd = to_dtype_bits(np.random.default_rng(601).standard_normal((nq, heads * D), dtype=np.float32), "bf16")
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="bf16") as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype="bf16")
        out = kv.AttentionChunk(0, pos0, qb, scale, q_dtype="bf16")
    for i in (0, 1, 31, 63, 64, 255, 1000, 1337, 2047):
        check_query(out[i], Kd[:pos0 + i + 1], Vd[:pos0 + i + 1], qd[i], heads, kv_heads, D, scale,
                    TOL_REL["bf16"], f"C3 query {i}")
    # every query: causal attention recomputed in fp32 on the CPU (batched per kv head; a
    # plain fp32 formulation agrees with the oracle's op order to ~1e-6, far inside the
    # tolerance), at the same tolerances, query by query
    check_all_queries(out, Kd, Vd, qd, heads, kv_heads, D, pos0, scale, TOL_REL["bf16"], "C3")


def check_all_queries(out, Kd, Vd, qd, heads, kv_heads, D, pos0, scale, tol_rel, what):
    import torch

    nq, n = qd.shape[0], Kd.shape[0]
    G = heads // kv_heads
    K = torch.from_numpy(Kd).view(n, kv_heads, D)
    V = torch.from_numpy(Vd).view(n, kv_heads, D)
    Q = torch.from_numpy(qd).view(nq, heads, D)
    got = torch.from_numpy(np.ascontiguousarray(out)).view(nq, heads, D)
    seen = torch.arange(n)[None, :] > (pos0 + torch.arange(nq))[:, None]  # [nq, n]: past the query's position
    worst_abs, worst_rel = 0.0, 0.0
    for kvh in range(kv_heads):
        q = Q[:, kvh * G:(kvh + 1) * G, :]                        # [nq, G, D]
        s = torch.matmul(q, K[:, kvh, :].T.contiguous()) * scale  # [nq, G, n]
        s.masked_fill_(seen[:, None, :], float("-inf"))
        want = torch.matmul(torch.softmax(s, dim=-1), V[:, kvh, :].contiguous())  # [nq, G, D]
        g = got[:, kvh * G:(kvh + 1) * G, :]
        d = (g - want).reshape(nq, -1)
        abs_err = d.abs().max(dim=1).values
        rel_err = d.norm(dim=1) / want.reshape(nq, -1).norm(dim=1)
        worst_abs, worst_rel = max(worst_abs, float(abs_err.max())), max(worst_rel, float(rel_err.max()))
        bad = torch.nonzero((abs_err > 1e-3) | (rel_err > tol_rel)).flatten()
        assert bad.numel() == 0, f"{what}: kv head {kvh}, query {int(bad[0])}: max-abs {float(abs_err[bad[0]]):.2e} rel {float(rel_err[bad[0]]):.2e}"
    print(f"{what}, all {nq} queries vs fp32 CPU attention: worst max-abs {worst_abs:.2e}, worst rel-L2 {worst_rel:.2e}")


def test_c4_speculative_verify_fp16(gpu):
    """64 q heads / 8 kv heads: 8 draft queries at 131072..131079 over fp16 KV, causal among drafts."""
    heads, kv_heads, D, pos0, nq = 64, 8, 128, 131072, 8
    n = pos0 + nq
    Kb, Kd, Vb, Vd = make(700, n, kv_heads * D, "f16")
    qb, qd = to_dtype_bits(np.random.default_rng(701).standard_normal((nq, heads * D), dtype=np.float32), "f16")
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="f16") as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype="f16")
        out = kv.AttentionChunk(0, pos0, qb, scale, q_dtype="f16")
        single = kv.Attention(0, pos0 + 3, qd[3], scale)
    for i in range(nq):
        check_query(out[i], Kd[:pos0 + i + 1], Vd[:pos0 + i + 1], qd[i], heads, kv_heads, D, scale,
                    TOL_REL["f16"], f"C4 verify draft {i}")
    assert_close(out[3], single, 1e-3, 1e-3, "verify draft 3 vs single decode call")


@pytest.mark.parametrize("dtype,heads,kv_heads,D,pos0,nq,q_dtype", [
    ("f16", 8, 8, 64, 0, 300, "f16"),        # prefill from scratch, group 1
    ("bf16", 16, 8, 128, 1000, 77, "bf16"),  # group 2, ragged query block
    ("f16", 64, 8, 128, 513, 40, "f32"),     # group 8, fp32 queries as hi + lo fp16
    ("bf16", 32, 4, 64, 255, 129, "bf16"),   # head_dim 64, crosses page boundaries
    ("f16", 4, 4, 128, 7, 1, "f16"),         # single query
    ("bf16", 32, 8, 128, 4000, 300, "f32"),  # fp32 queries as hi + lo bf16, two N tiles
    ("bf16", 8, 2, 64, 130, 1000, "f16"),    # fp16 queries into a bf16 cache, four N tiles
    ("f16", 16, 2, 128, 70000, 5, "f16"),    # few queries over a long cache: split-K, 3 stages
    # verify-sized blocks (one N tile: two waves per row group, one per 32-position half)
    ("f16", 64, 8, 64, 20, 8, "f32"),        # one tile of 28 positions: the second half all masked
                                             # (fp16: over 21 keys bf16's 8-bit P alone errs ~1.6e-3)
    ("f16", 32, 8, 128, 40, 8, "f16"),       # one tile of 48: the drafts' causal edge in the second half
    ("bf16", 64, 8, 128, 100, 8, "bf16"),    # two tiles, the last one partial
    ("bf16", 64, 8, 128, 5000, 8, "f32"),    # fp32 drafts as hi + lo bf16 over split keys
])
def test_chunk_mfma_shapes(gpu, dtype, heads, kv_heads, D, pos0, nq, q_dtype):
    n = pos0 + nq
    Kb, Kd, Vb, Vd = make(n + heads, n, kv_heads * D, dtype)
    qb, qd = to_dtype_bits(np.random.default_rng(n).standard_normal((nq, heads * D), dtype=np.float32), q_dtype)
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n + 10, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        out = kv.AttentionChunk(0, pos0, qb, scale, q_dtype=q_dtype)
    for i in sorted({0, nq // 2, nq - 1}):
        check_query(out[i], Kd[:pos0 + i + 1], Vd[:pos0 + i + 1], qd[i], heads, kv_heads, D, scale,
                    TOL_REL[dtype], f"{dtype} H{heads}/Hkv{kv_heads}/D{D} pos0 {pos0} query {i}")
