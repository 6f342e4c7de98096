"""GPU parity of the fused RoPE + append step (StreamingEngine.cs:245-248:
TransformerOps.BuildCosSinInto / Rope, TransformerOps.cs:56-88, then PagedKvCache.Append).

The oracle restates the rotation with glibc powf/cosf/sinf in the reference's fp32
order; the library takes the same host powf for the frequencies and the device cosf/
sinf, so rotated values agree to a few fp32 ulps (tolerance: |diff| <= 4e-6 * max|x| +
1e-7 for fp32 rows; 16-bit caches: every stored element within one 16-bit ulp plus that
fp32 tolerance of the oracle's rounding, and at least 99% of them bit-identical).  The reference's own RopeTest
(Tests/Program.cs:282-306) is checked through the GPU.
"""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.util import assert_close, normal

pytestmark = pytest.mark.gpu


def rope_ref(x, D, pos0, theta):
    return oracle.rope_rows(np.array(x, dtype=np.float32, copy=True), D, pos0, theta)


def close_rows(got, want, what):
    tol = 4e-6 * float(np.max(np.abs(want))) + 1e-7
    err = float(np.max(np.abs(got - want)))
    print(f"{what}: max-abs {err:.2e} (tolerance {tol:.2e})")
    assert err <= tol, what


def test_reference_rope_test_norm_through_gpu(gpu):
    """Tests/Program.cs:282-306: theta 10000, pos 123, the rotation keeps each head's norm (1e-4)."""
    heads, kv_heads, D = 4, 2, 64
    q = normal(300, heads * D)
    k, v = normal(301, kv_heads * D), normal(302, kv_heads * D)
    with qr.PagedKvCache(1, heads, kv_heads, D, 256) as kv:
        qr_ = kv.AppendRope(0, 123, q, k, v, 10000.0)
        kr, vr = kv.Read(0, 123, 1)
    for h in range(heads):
        assert abs(np.linalg.norm(qr_[h * D:(h + 1) * D]) - np.linalg.norm(q[h * D:(h + 1) * D])) <= 1e-4
    for h in range(kv_heads):
        assert abs(np.linalg.norm(kr[0, h * D:(h + 1) * D]) - np.linalg.norm(k[h * D:(h + 1) * D])) <= 1e-4
    assert np.array_equal(vr[0], v)


@pytest.mark.parametrize("theta,pos0,n", [(10000.0, 0, 300), (500000.0, 131000, 72)])
def test_rope_append_matches_oracle_fp32(gpu, theta, pos0, n):
    heads, kv_heads, D = 8, 2, 128
    Q = normal(310 + n, (n, heads * D))
    K, V = normal(311 + n, (n, kv_heads * D)), normal(312 + n, (n, kv_heads * D))
    with qr.PagedKvCache(1, heads, kv_heads, D, pos0 + n) as kv:
        qs = [kv.AppendRope(0, pos0 + t, Q[t], K[t], V[t], theta) for t in range(min(n, 40))]
        kr, vr = kv.Read(0, pos0, min(n, 40))
    close_rows(np.stack(qs), rope_ref(Q[:40], D, pos0, theta), f"q host path theta {theta}")
    close_rows(kr, rope_ref(K[:40], D, pos0, theta), f"k host path theta {theta}")
    assert np.array_equal(vr, V[:40])


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_rope_append_dev_bulk(gpu, dtype):
    """n positions in one device call, C2 head geometry and theta 5e5, positions near 32K."""
    import torch
    heads, kv_heads, D, pos0, n = 32, 8, 128, 32000, 768
    Q = normal(320, (n, heads * D))
    K, V = normal(321, (n, kv_heads * D)), normal(322, (n, kv_heads * D))
    theta = 500000.0
    dev = torch.device("cuda")
    qd = torch.from_numpy(Q).to(dev)
    with qr.PagedKvCache(1, heads, kv_heads, D, pos0 + n, kv_dtype=dtype) as kv:
        kv.AppendRopeDev(0, pos0, qd, torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), theta)
        torch.cuda.synchronize()
        kr, vr = kv.Read(0, pos0, n)
        assert kv.SeqLen == pos0 + n
    qw, kw = rope_ref(Q, D, pos0, theta), rope_ref(K, D, pos0, theta)
    close_rows(qd.cpu().numpy(), qw, "q rotated in place")
    if dtype == "f32":
        close_rows(kr, kw, "k pages")
        assert np.array_equal(vr, V)
        return
    enc = oracle.f32_to_f16 if dtype == "f16" else oracle.f32_to_bf16
    dec = oracle.f16_to_f32 if dtype == "f16" else oracle.bf16_to_f32
    assert np.array_equal(vr, enc(V))
    same = np.mean(kr == enc(kw))
    # one 16-bit ulp, plus the fp32 rotation difference (a few fp32 ulps of the inputs),
    # which near zero spans several 16-bit subnormal steps
    ulp = (2.0 ** -10 if dtype == "f16" else 2.0 ** -7) * np.maximum(np.abs(kw), 2.0 ** -14)
    diff = np.abs(dec(kr) - dec(enc(kw)))
    print(f"{dtype}: largest difference {diff.max():.2e}")
    assert np.all(diff <= ulp * 1.01 + 4e-6 * float(np.max(np.abs(kw)))), "beyond one 16-bit ulp"
    print(f"{dtype}: {100 * same:.3f}% of rotated K elements bit-identical to the oracle's rounding")
    assert same >= 0.99


@pytest.mark.parametrize("dtype,D", [("f16", 128), ("bf16", 128), ("f16", 64), ("bf16", 64), ("f16", 80),
                                     ("bf16", 96)])
def test_rope_append_dev_ragged_ranges(gpu, dtype, D):
    """Device appends at unaligned positions and lengths (single rows, runs that end
    mid-chunk, runs across page boundaries): every V row read back equals its 16-bit
    rounding, so no append overwrote a neighbour's slots, and K agrees as in the bulk test."""
    import torch
    heads, kv_heads, theta = 4, 2, 10000.0
    spans = [(0, 37), (37, 1), (38, 3), (41, 300), (341, 171), (512, 8), (520, 1), (521, 250)]
    total = spans[-1][0] + spans[-1][1]
    Q = normal(340 + D, (total, heads * D))
    K, V = normal(341 + D, (total, kv_heads * D)), normal(342 + D, (total, kv_heads * D))
    dev = torch.device("cuda")
    with qr.PagedKvCache(1, heads, kv_heads, D, total, kv_dtype=dtype) as kv:
        for pos0, n in spans:
            qd = torch.from_numpy(Q[pos0:pos0 + n]).to(dev)
            kv.AppendRopeDev(0, pos0, qd, torch.from_numpy(K[pos0:pos0 + n]).to(dev),
                             torch.from_numpy(V[pos0:pos0 + n]).to(dev), theta)
        torch.cuda.synchronize()
        kr, vr = kv.Read(0, 0, total)
    enc = oracle.f32_to_f16 if dtype == "f16" else oracle.f32_to_bf16
    bad = np.argwhere(vr != enc(V))
    assert bad.size == 0, f"V differs at (position, column) {tuple(bad[0])}, {len(bad)} elements"
    kw = rope_ref(K, D, 0, theta)
    assert np.mean(kr == enc(kw)) >= 0.99


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rope_append_dev_without_q_across_a_page(gpu, dtype):
    """K and V only (no q rows): positions 250..286 cross the page boundary at 256 and two
    32-position V tiles, both partial; rows before and after stay untouched."""
    import torch
    heads, kv_heads, D, pos0, n, theta = 8, 2, 128, 250, 37, 500000.0
    K, V = normal(350, (n, kv_heads * D)), normal(351, (n, kv_heads * D))
    K0, V0 = normal(352, (pos0, kv_heads * D)), normal(353, (pos0, kv_heads * D))
    dev = torch.device("cuda")
    with qr.PagedKvCache(1, heads, kv_heads, D, 320, kv_dtype=dtype) as kv:
        kv.AppendRopeDev(0, 0, None, torch.from_numpy(K0).to(dev), torch.from_numpy(V0).to(dev), theta)
        kv.AppendRopeDev(0, pos0, None, torch.from_numpy(K).to(dev), torch.from_numpy(V).to(dev), theta)
        torch.cuda.synchronize()
        kr, vr = kv.Read(0, 0, pos0 + n)
        assert kv.SeqLen == pos0 + n
    enc = oracle.f32_to_f16 if dtype == "f16" else oracle.f32_to_bf16
    assert np.array_equal(vr, enc(np.concatenate([V0, V])))
    kw = np.concatenate([rope_ref(K0, D, 0, theta), rope_ref(K, D, pos0, theta)])
    assert np.mean(kr == enc(kw)) >= 0.99


def test_rope_append_then_attention(gpu):
    """Decode over rows appended through the fused step equals the oracle's attention over
    oracle-rotated rows (fp32 accumulation tolerance)."""
    heads, kv_heads, D, n, theta = 8, 2, 64, 700, 10000.0
    Q = normal(330, (n, heads * D))
    K, V = normal(331, (n, kv_heads * D)), normal(332, (n, kv_heads * D))
    with qr.PagedKvCache(1, heads, kv_heads, D, n) as kv:
        for t in range(n - 1):
            kv.AppendRope(0, t, Q[t], K[t], V[t], theta)
        qlast = kv.AppendRope(0, n - 1, Q[n - 1], K[n - 1], V[n - 1], theta)
        got = kv.Attention(0, n - 1, qlast, 1 / math.sqrt(D))
    Kw = rope_ref(K, D, 0, theta)
    qw = rope_ref(Q[n - 1:], D, n - 1, theta)[0]
    want = oracle.kv_attention(Kw, V, qw, heads, kv_heads, D, 1 / math.sqrt(D))
    assert_close(got, want, 1e-3, 1e-4, "attention after fused RoPE + append")


def test_rope_append_errors(gpu):
    with qr.PagedKvCache(1, 4, 2, 64, 100) as kv:
        with pytest.raises(qr.QrOutOfRange):
            kv.AppendRope(0, 100, np.zeros(256, np.float32), np.zeros(128, np.float32), np.zeros(128, np.float32), 1e4)
        with pytest.raises(ValueError):
            kv.AppendRope(0, 1, np.zeros(255, np.float32), np.zeros(128, np.float32), np.zeros(128, np.float32), 1e4)
        with pytest.raises(qr.QrInvalidArgument):
            kv.AppendRope(3, 1, np.zeros(256, np.float32), np.zeros(128, np.float32), np.zeros(128, np.float32), 1e4)
