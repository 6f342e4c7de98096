"""GPU parity of the MLA absorbed path (MlaLatentCache.cs:29-65, StreamingEngine.cs:508-577).

Tolerances: fp32 latents (generic kernel, fp32 accumulation): max-abs <= 1e-3,
rel-L2 <= 1e-4.  16-bit latents on MFMA tiles (operands in the cache's 16-bit type,
q~ as hi + lo parts, P rounded to the cache type, fp32 accumulation): max-abs <= 1e-3,
rel-L2 <= 5e-3 against the oracle fed the same 16-bit latent values; for latents far
from unit scale the max-abs bound is 1e-3 times the largest output magnitude.  Both
sides' errors against fp64 are printed.
"""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from oracle import oracle
from tests.util import assert_close, errors, normal, to_dtype_bits

pytestmark = pytest.mark.gpu


def check_mla(got, lat, qt, qrp, kv_lora, rope, scale, tol_rel, what):
    want = oracle.mla_attention(lat, qt, qrp, kv_lora, rope, scale)
    a, r = assert_close(got, want, 1e-3, tol_rel, what)
    f64 = oracle.mla_attention_f64(lat, qt, qrp, kv_lora, rope, scale)
    print(f"{what}: vs oracle max-abs {a:.2e} rel {r:.2e} | vs fp64: gpu {errors(got, f64)[1]:.2e} "
          f"oracle {errors(want, f64)[1]:.2e}")


def run_mla(dtype, heads, kv_lora, rope, n, pos=None, seed=0, layers=1, layer=0):
    lat = normal(seed, (n, kv_lora + rope))
    bits, latd = to_dtype_bits(lat, dtype)
    qt = normal(seed + 1, (heads, kv_lora))
    qrp = normal(seed + 2, (heads, rope)) if rope else np.zeros((heads, 0), np.float32)
    scale = 1 / math.sqrt(192)
    with qr.MlaLatentCache(layers, kv_lora + rope, n, dtype=dtype, rope=rope) as m:
        m.AppendRange(layer, 0, bits, src_dtype=dtype)
        p = n - 1 if pos is None else pos
        got = m.AbsorbedAttention(layer, p, qt, qrp, scale)
    return got, latd[:p + 1], qt, qrp, scale


def test_c5_mla_absorbed_decode_16k_bf16(gpu):
    """128 heads, 512 + 64 latent, 16,384 bf16 latent tokens (64 pages), scale 1/sqrt(192)."""
    got, lat, qt, qrp, s = run_mla("bf16", 128, 512, 64, 16384, seed=10)
    check_mla(got, lat, qt, qrp, 512, 64, s, 5e-3, "C5 bf16")


@pytest.mark.parametrize("dtype,heads,rope,n,pos", [
    ("f16", 128, 64, 3000, None),
    ("bf16", 40, 64, 1000, None),     # heads not a multiple of 64, ragged last tile
    ("bf16", 64, 0, 700, None),       # NoPE latent (GLM-5.3-Flash style)
    ("f16", 16, 64, 777, 31),         # fewer positions than one tile
    ("bf16", 128, 64, 600, 0),        # one position: u = c_0 exactly up to fp16 rounding
    ("bf16", 8, 64, 500, None),       # fewer heads than one 32-head group
    ("f16", 33, 0, 1300, None),       # one head past a group boundary
    ("bf16", 128, 64, 9000, 5000),    # mid-sequence position, rows past it resident
])
def test_mla_mfma_shapes(gpu, dtype, heads, rope, n, pos):
    got, lat, qt, qrp, s = run_mla(dtype, heads, 512, rope, n, pos=pos, seed=n)
    check_mla(got, lat, qt, qrp, 512, rope, s, 5e-3, f"{dtype} H{heads} rope{rope} n{n} pos{pos}")


@pytest.mark.parametrize("heads,kv_lora,rope,n", [(16, 512, 64, 700), (4, 8, 0, 10), (3, 96, 32, 300)])
def test_mla_fp32_generic(gpu, heads, kv_lora, rope, n):
    got, lat, qt, qrp, s = run_mla("f32", heads, kv_lora, rope, n, seed=heads + n)
    check_mla(got, lat, qt, qrp, kv_lora, rope, s, 1e-4, f"f32 H{heads} lora{kv_lora} rope{rope} n{n}")


@pytest.mark.parametrize("rope", [0, 16])
def test_mla_absorbed_equals_expanded_through_gpu(gpu, rope):
    """Cli/Commands.cs:2065-2152: q-absorb -> GPU latent attention -> W_UV equals the
    expanded fp64 attention (H4, kvLora 8, nope 4, v 4, seq 10; plus a rope case)."""
    heads, kv_lora, nope, vdim, seq = 4, 8, 4, 4, 10
    rng = np.random.default_rng(29 + rope)
    R = lambda n: (rng.random(n) * 2 - 1).astype(np.float32)  # noqa: E731
    q = R(heads * (nope + rope))
    kvb = R(heads * (nope + vdim) * kv_lora)
    lat = R(seq * (kv_lora + rope)).reshape(seq, kv_lora + rope)
    scale = 1 / math.sqrt(nope + rope)
    qt = oracle.mla_q_absorb(q, kvb, heads, nope, rope, vdim, kv_lora)
    qrp = q.reshape(heads, nope + rope)[:, nope:]
    with qr.MlaLatentCache(1, kv_lora + rope, 64, rope=rope) as m:
        for t in range(seq):
            m.Append(0, t, lat[t])
        u = m.AbsorbedAttention(0, seq - 1, qt, qrp, scale)
    out = oracle.mla_wuv(u, kvb, heads, nope, vdim, kv_lora)
    want = oracle.mla_expanded_f64(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale)
    assert np.max(np.abs(out - want)) <= 1e-4


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_mla_reference_constructor_and_late_split(gpu, dtype):
    """new MlaLatentCache(layers, latentDim, maxSeq) as StreamingEngine.cs:96-97 calls it:
    appends need the row width only; attention needs the kv_lora/rope split, which MlaLayer
    supplies (SetRope); the result equals a cache created with the split."""
    kv_lora, rope, n, heads = 512, 64, 700, 16
    lat = normal(31, (n, kv_lora + rope))
    bits, _ = to_dtype_bits(lat, dtype)
    qt, qrp = normal(32, (heads, kv_lora)), normal(33, (heads, rope))
    with qr.MlaLatentCache(1, kv_lora + rope, 1000, dtype=dtype) as m, \
            qr.MlaLatentCache(1, kv_lora + rope, 1000, dtype=dtype, rope=rope) as ref:
        assert m.max_seq() == 1000
        m.AppendRange(0, 0, bits, src_dtype=dtype)
        ref.AppendRange(0, 0, bits, src_dtype=dtype)
        with pytest.raises(qr.QrInvalidArgument):
            m.AbsorbedAttention(0, n - 1, qt, qrp, 0.07)
        with pytest.raises(qr.QrInvalidArgument):
            m.SetRope(kv_lora + rope)              # no room for kv_lora
        m.SetRope(rope)
        assert np.array_equal(m.AbsorbedAttention(0, n - 1, qt, qrp, 0.07),
                              ref.AbsorbedAttention(0, n - 1, qt, qrp, 0.07))


def test_mla_cache_state(gpu):
    """Paging, Page() copy-out, BytesUsed, Truncate/Reset (MlaLatentCache.cs:29-65)."""
    kv_lora, rope, n = 512, 64, 600
    lat = normal(5, (n, kv_lora + rope))
    bits = oracle.f32_to_bf16(lat)
    with qr.MlaLatentCache(2, kv_lora + rope, 1024, dtype="bf16", rope=rope) as m:
        for t in range(300):
            m.Append(1, t, lat[t])          # fp32 rows through the reference codec
        m.AppendRange(1, 300, bits[300:], src_dtype="bf16")
        assert m.SeqLen == n and m.PageCount(1) == 3 and m.PageCount(0) == 0
        assert m.BytesUsed == 3 * 256 * (kv_lora + rope) * 2
        page1 = m.Page(1, 1)
        assert np.array_equal(page1[:n - 256 if n < 512 else 256], oracle.bf16_to_f32(bits[256:512]))
        m.Truncate(100)
        assert m.SeqLen == 100
        m.Reset()
        assert m.SeqLen == 0 and m.BytesUsed == 3 * 256 * (kv_lora + rope) * 2
        with pytest.raises(qr.QrNotResident):
            m.AbsorbedAttention(0, 0, normal(1, (8, kv_lora)), normal(2, (8, rope)), 0.1)
        with pytest.raises(qr.QrOutOfRange):
            m.Append(1, 1024, lat[0])
        with pytest.raises(qr.QrOutOfRange):
            m.Append(1, 0, np.zeros(kv_lora + rope + 1, np.float32))
        with pytest.raises(qr.QrInvalidArgument):
            m.AbsorbedAttention(1, 10, normal(1, (300, kv_lora)), normal(2, (300, rope)), 0.1)


def test_mla_rows_past_pos_are_not_read_into_the_result(gpu):
    """Rows after pos hold NaN; attention at pos sees rows 0..pos only (seq = pos + 1)."""
    n, pos, heads = 700, 300, 64
    lat = normal(77, (n, 576))
    bits, latd = to_dtype_bits(lat, "bf16")
    bits = bits.copy()
    bits[pos + 1:] = 0x7FC0  # bf16 quiet NaN
    qt, qrp = normal(78, (heads, 512)), normal(79, (heads, 64))
    scale = 1 / math.sqrt(192)
    with qr.MlaLatentCache(1, 576, n, dtype="bf16", rope=64) as m:
        m.AppendRange(0, 0, bits, src_dtype="bf16")
        got = m.AbsorbedAttention(0, pos, qt, qrp, scale)
    assert np.isfinite(got).all()
    check_mla(got, latd[:pos + 1], qt, qrp, 512, 64, scale, 5e-3, "NaN rows past pos")


def test_mla_dev_entry_with_unaligned_queries(gpu):
    """The device entry point accepts q~ / q_rope views that are not 16-byte aligned."""
    import torch
    n, heads = 1500, 40
    lat = normal(81, (n, 576))
    bits, latd = to_dtype_bits(lat, "bf16")
    qt, qrp = normal(82, (heads, 512)), normal(83, (heads, 64))
    scale = 1 / math.sqrt(192)
    dev = torch.device("cuda")
    qt_buf = torch.zeros(heads * 512 + 1, dtype=torch.float32, device=dev)
    qr_buf = torch.zeros(heads * 64 + 3, dtype=torch.float32, device=dev)
    qt_buf[1:] = torch.from_numpy(qt.ravel()).to(dev)
    qr_buf[3:] = torch.from_numpy(qrp.ravel()).to(dev)
    u = torch.empty(heads * 512, dtype=torch.float32, device=dev)
    with qr.MlaLatentCache(1, 576, n, dtype="bf16", rope=64) as m:
        m.AppendRange(0, 0, bits, src_dtype="bf16")
        m.AbsorbedAttentionDev(0, n - 1, qt_buf[1:], qr_buf[3:], u, scale)
        torch.cuda.synchronize()
        aligned = m.AbsorbedAttention(0, n - 1, qt, qrp, scale)
    got = u.cpu().numpy().reshape(heads, 512)
    assert np.array_equal(got, aligned)
    check_mla(got, latd, qt, qrp, 512, 64, scale, 5e-3, "unaligned q")


@pytest.mark.parametrize("case", ["spikes", "all_large", "all_tiny"])
def test_mla_bf16_latents_outside_the_fp16_range(gpu, case):
    """bf16 latents hold any finite fp32 exponent (the reference keeps fp32 latents,
    MlaLatentCache.cs:45-51, StreamingEngine.cs:531-568): elements at +-1e5 and +-1e-6
    among N(0,1) ones, a whole cache scaled by 1e6 (outputs far past fp16's 65504, with
    several splits), and one scaled by 1e-6 (fp16 subnormals).  The spiked columns get a
    zero query weight, so the 1e5 values pass through every QK product (an fp16 operand
    would turn them into inf, and inf * 0 into NaN) and through the latent sum, while the
    scores stay well conditioned (a score of 1e4 would make the softmax depend on its
    last bits, beyond what either fp32 side resolves)."""
    heads, kv_lora, rope, n = 128, 512, 64, 4096
    rng = np.random.default_rng(1234)
    lat = rng.standard_normal((n, kv_lora + rope), dtype=np.float32)
    qt = rng.standard_normal((heads, kv_lora), dtype=np.float32)
    qrp = rng.standard_normal((heads, rope), dtype=np.float32)
    if case == "spikes":
        cols = rng.choice(kv_lora + rope, 24, replace=False)
        for k, val in enumerate((1e5, -1e5, 1e-6, -1e-6)):
            lat[rng.integers(0, n, 40), np.repeat(cols[6 * k:6 * k + 6], 40 // 6 + 1)[:40]] = val
        qt[:, cols[cols < kv_lora]] = 0.0
        qrp[:, cols[cols >= kv_lora] - kv_lora] = 0.0
    elif case == "all_large":
        lat *= 1e6
        qt *= 1e-6
        qrp *= 1e-6
    else:
        lat *= 1e-6
        qt *= 1e6
        qrp *= 1e6
    bits, latd = to_dtype_bits(lat, "bf16")
    scale = 1 / math.sqrt(192)
    with qr.MlaLatentCache(1, kv_lora + rope, n, dtype="bf16", rope=rope) as m:
        m.AppendRange(0, 0, bits, src_dtype="bf16")
        got = m.AbsorbedAttention(0, n - 1, qt, qrp, scale)
    want = oracle.mla_attention(latd, qt, qrp, kv_lora, rope, scale)
    assert np.isfinite(got).all(), f"{case}: non-finite output"
    a, r = assert_close(got, want, 1e-3 * max(1.0, float(np.max(np.abs(want)))), 5e-3, f"bf16 range {case}")
    f64 = oracle.mla_attention_f64(latd, qt, qrp, kv_lora, rope, scale)
    print(f"bf16 range {case}: max |u| {np.max(np.abs(want)):.3e}, vs oracle max-abs {a:.2e} rel {r:.2e} | "
          f"vs fp64: gpu {errors(got, f64)[1]:.2e} oracle {errors(want, f64)[1]:.2e}")
