"""PagedKvCache with head sizes the vector and MFMA kernels do not take (not a multiple of 8,
or outside 16..256): the reference accepts any headDim (PagedKvCache.cs:29-37; DotF32 and
AxpyF32 with their scalar tails, SimdMath.cs:36-71; RoPE over the pairs i < headDim/2,
TransformerOps.cs:56-88).  These run on the scalar generic kernels; parity against the
oracle at the decode tolerances (max-abs <= 1e-3, relative L2 <= 1e-4 on exactly decoded
KV) and the RoPE tolerances of test_gpu_rope_append.py."""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.test_gpu_decode import check_decode
from tests.test_gpu_rope_append import close_rows, rope_ref
from tests.util import normal, to_dtype_bits

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,heads,kv_heads,D,seq", [
    ("f32", 4, 2, 1, 300),
    ("f32", 6, 3, 7, 700),
    ("f16", 4, 4, 12, 513),
    ("bf16", 8, 2, 17, 5000),    # splits merged by the generic merge
    ("f32", 5, 2, 100, 2100),    # kv_heads does not divide heads
    ("f16", 4, 1, 300, 1500),
    ("f32", 2, 2, 512, 600),
    ("bf16", 4, 2, 8, 260),
])
def test_decode_any_head_dim(gpu, dtype, heads, kv_heads, D, seq):
    """Full and partial lengths; rows past the attended position hold NaN, so a read past
    the row or past the position would show."""
    q = normal(seq + D, heads * D)
    Kb, K = to_dtype_bits(normal(seq + D + 1, (seq, kv_heads * D)), dtype)
    Vb, V = to_dtype_bits(normal(seq + D + 2, (seq, kv_heads * D)), dtype)
    if dtype == "f32":
        nanb = np.full((40, kv_heads * D), np.nan, np.float32)
    else:
        nanb = np.full((40, kv_heads * D), 0x7E00 if dtype == "f16" else 0x7FC0, np.uint16)
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, seq + 40, kv_dtype=dtype) as kv:
        kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype)
        kv.AppendRange(0, seq, nanb, nanb, src_dtype=dtype)
        kr, vr = kv.Read(0, 0, seq)
        assert np.array_equal(kr, Kb) and np.array_equal(vr, Vb)
        for p in (seq - 1, seq // 3, 0):
            got = kv.Attention(0, p, q, scale)
            assert np.isfinite(got).all()
            check_decode(got, K[:p + 1], V[:p + 1], q, heads, kv_heads, D, scale, f"{dtype} H{heads}/{kv_heads} D{D} pos {p}")


def test_batch_chunk_and_device_paths_any_head_dim(gpu):
    """Batched entries with their own lengths, causal chunk queries (one decode entry per
    query), device-position steps and the no-allocation entry point at head_dim 17."""
    import torch
    heads, kv_heads, D, n = 6, 2, 17, 3000
    K, V = normal(700, (n, kv_heads * D)), normal(701, (n, kv_heads * D))
    qs = normal(702, (4, heads * D))
    dev = torch.device("cuda")
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="f32", max_batch=2) as kv:
        kv.AppendRange(0, 0, K, V)
        kv.AppendRange(0, 0, K[:1000] * 0.5, V[:1000], seq_id=1)
        out = kv.AttentionBatch(0, [0, 1, 0], [n - 1, 999, 40], qs[:3], 0.3)
        check_decode(out[0], K, V, qs[0], heads, kv_heads, D, 0.3, "batch entry 0")
        check_decode(out[1], K[:1000] * 0.5, V[:1000], qs[1], heads, kv_heads, D, 0.3, "batch entry 1")
        check_decode(out[2], K[:41], V[:41], qs[2], heads, kv_heads, D, 0.3, "batch entry 2")
        ch = kv.AttentionChunk(0, n - 4, qs, 0.3)
        for i in range(4):
            check_decode(ch[i], K[:n - 3 + i], V[:n - 3 + i], qs[i], heads, kv_heads, D, 0.3, f"chunk query {i}")
        qd = torch.from_numpy(qs[:1]).to(dev)
        o1 = torch.empty_like(qd)
        o2 = torch.empty_like(qd)
        pos = torch.tensor([1234], dtype=torch.int32, device=dev)
        kv.AttentionStepDev(0, [0], pos, qd, o1, 0.3)
        kv.AttentionDevNoAlloc(0, [0], [1234], qd, o2, 0.3)
        torch.cuda.synchronize()
        check_decode(o1.cpu().numpy()[0], K[:1235], V[:1235], qs[0], heads, kv_heads, D, 0.3, "device position")
        check_decode(o2.cpu().numpy()[0], K[:1235], V[:1235], qs[0], heads, kv_heads, D, 0.3, "no-allocation call")


@pytest.mark.parametrize("dtype,D", [("f32", 1), ("f32", 7), ("f16", 17), ("bf16", 100), ("f32", 300), ("f16", 512)])
def test_rope_append_any_head_dim(gpu, dtype, D):
    """Host and device RoPE appends: pairs (i, i + D/2) rotated, dim D - 1 of an odd head
    size left as it was (as the reference's RopeHead), q rotated in place."""
    import torch
    heads, kv_heads, theta, pos0, n = 4, 2, 10000.0, 250, 20
    Q = normal(720 + D, (n, heads * D))
    K, V = normal(721 + D, (n, kv_heads * D)), normal(722 + D, (n, kv_heads * D))
    dev = torch.device("cuda")
    with qr.PagedKvCache(1, heads, kv_heads, D, pos0 + 2 * n, kv_dtype=dtype) as kv:
        qh = np.stack([kv.AppendRope(0, pos0 + t, Q[t], K[t], V[t], theta) for t in range(n)])
        qd = torch.from_numpy(Q).to(dev)
        kv.AppendRopeDev(0, pos0 + n, qd, torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), theta)
        torch.cuda.synchronize()
        kr, vr = kv.Read(0, pos0, 2 * n)
    qw, kw = rope_ref(Q, D, pos0, theta), rope_ref(K, D, pos0, theta)
    qw2, kw2 = rope_ref(Q, D, pos0 + n, theta), rope_ref(K, D, pos0 + n, theta)
    close_rows(qh, qw, f"q host D{D}")
    close_rows(qd.cpu().numpy(), qw2, f"q device D{D}")
    if D % 2:
        last = np.arange(heads) * D + D - 1
        assert np.array_equal(qh[:, last], Q[:, last]), "odd head size: the last dim stays"
    if dtype == "f32":
        close_rows(kr[:n], kw, f"k host D{D}")
        close_rows(kr[n:], kw2, f"k device D{D}")
        assert np.array_equal(vr, np.concatenate([V, V]))
        return
    enc = oracle.f32_to_f16 if dtype == "f16" else oracle.f32_to_bf16
    assert np.array_equal(vr, enc(np.concatenate([V, V])))
    assert np.mean(kr == enc(np.concatenate([kw, kw2]))) >= 0.99


def test_rope_step_dev_any_head_dim(gpu):
    """Device-position RoPE append (page claim on the GPU) at head_dim 21, then decode."""
    import torch
    heads, kv_heads, D, theta, n = 4, 2, 21, 500000.0, 300
    Q = normal(740, (n, heads * D))
    K, V = normal(741, (n, kv_heads * D)), normal(742, (n, kv_heads * D))
    dev = torch.device("cuda")
    with qr.PagedKvCache(1, heads, kv_heads, D, 512) as kv:
        pos = torch.zeros(1, dtype=torch.int32, device=dev)
        qd = torch.from_numpy(Q).to(dev)
        kd, vd = torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev)
        for t in range(n):
            pos.fill_(t)
            kv.AppendRopeStepDev(0, pos, qd[t], kd[t], vd[t], theta)
        torch.cuda.synchronize()
        assert kv.SeqLen == n
        kr, vr = kv.Read(0, 0, n)
        close_rows(kr, rope_ref(K, D, 0, theta), "k rows")
        assert np.array_equal(vr, V)
        qlast = qd[n - 1].cpu().numpy()
        check_decode(kv.Attention(0, n - 1, qlast, 0.2), kr, vr, qlast, heads, kv_heads, D, 0.2, "decode after steps")
