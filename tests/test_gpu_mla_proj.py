"""GPU parity of the MLA projections either side of the absorbed attention
(StreamingEngine.cs:517-529 q-absorb, :569-576 W_UV) with on-the-fly dequant of the
kvb rows (BlockDequantizer.Dequantize).

Bar: bit-exact.  Both projections follow the reference's fp32 operation order
(sequential multiply-then-add over j for the absorb, SimdMath.DotF32's 8 lane sums and
lane-order HSum for W_UV), and the decoders reproduce the reference's roundings, so
the GPU must equal the oracle exactly for every format.  The whole layer block
(qr_mla_attend_absorbed) inherits the attention kernel's tolerance (16-bit latents:
max-abs <= 1e-3, rel-L2 <= 5e-3).
"""
import math

import numpy as np
import pytest
import torch

import qauntrunner_amd as qr
from oracle import oracle
from tests import quant
from tests.util import assert_close, errors, normal, to_dtype_bits

pytestmark = pytest.mark.gpu

FORMATS = ["F32", "F16", "BF16", "Q4_0", "Q8_0", "Q4_K", "Q6_K"]


def kvb_rows(fmt, heads, nope, vdim, kv_lora, seed):
    """Seeded kvb weights in fmt: (raw uint8 [rows][row_bytes], decoded fp32 [rows][kv_lora])."""
    return quant.random_rows(quant.FMT[fmt], heads * (nope + vdim), kv_lora, seed)


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).cuda()


def run_proj(fmt, heads, nope, rope, vdim, kv_lora, nq, seed=0):
    raw, w = kvb_rows(fmt, heads, nope, vdim, kv_lora, seed)
    q = normal(seed + 1, (nq, heads, nope + rope))
    u = normal(seed + 2, (nq, heads, kv_lora))
    kvb = dev(raw.reshape(-1))
    qt = torch.empty((nq, heads, kv_lora), dtype=torch.float32, device="cuda")
    out = torch.empty((nq, heads, vdim), dtype=torch.float32, device="cuda")
    code = quant.FMT[fmt]
    qr.mla_q_absorb_dev(kvb, code, heads, nope, rope, vdim, kv_lora, dev(q), qt)
    qr.mla_wuv_dev(kvb, code, heads, nope, vdim, kv_lora, dev(u), out)
    torch.cuda.synchronize()
    want_qt = np.stack([oracle.mla_q_absorb(q[b], w, heads, nope, rope, vdim, kv_lora) for b in range(nq)])
    want_out = np.stack([oracle.mla_wuv(u[b], w, heads, nope, vdim, kv_lora) for b in range(nq)])
    return qt.cpu().numpy(), want_qt, out.cpu().numpy(), want_out


def assert_exact(got, want, what):
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ, first at {bad[0]}: "
                           f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_projections_bit_exact_per_format(gpu, fmt):
    """32 heads, nope 128, rope 64, vdim 128, kv_lora 512: both projections equal the oracle."""
    qt, want_qt, out, want_out = run_proj(fmt, 32, 128, 64, 128, 512, 1, seed=quant.FMT[fmt])
    assert_exact(qt, want_qt, f"{fmt} absorb")
    assert_exact(out, want_out, f"{fmt} W_UV")


def test_projections_c5_shape_bf16(gpu):
    """The GLM/DeepSeek layer shape: 128 heads, nope 128, vdim 128, kv_lora 512."""
    qt, want_qt, out, want_out = run_proj("BF16", 128, 128, 64, 128, 512, 1, seed=50)
    assert_exact(qt, want_qt, "C5 absorb")
    assert_exact(out, want_out, "C5 W_UV")


@pytest.mark.parametrize("fmt,heads,nope,rope,vdim,kv_lora,nq", [
    ("F32", 4, 20, 8, 40, 1024, 1),     # nope past the unroll, vdim past a row tile, two f32 slabs
    ("BF16", 5, 16, 0, 32, 8, 3),       # smallest kv_lora, NoPE, batch tile of 3
    ("Q8_0", 3, 7, 16, 33, 64, 5),      # 68-byte rows (dword staging), two batch tiles
    ("Q4_0", 2, 9, 4, 17, 32, 2),       # one 20-byte block per row
    ("Q6_K", 3, 10, 8, 20, 256, 1),     # 210-byte rows (2-byte staging)
    ("Q4_K", 2, 33, 64, 64, 1024, 4),   # four super-blocks per row
    ("F16", 16, 128, 64, 128, 512, 9),  # batch of 9 queries: tiles of 4, 4, 1
    ("BF16", 3, 36, 8, 16, 128, 2),     # nope past a whole number of 8-row DMA gathers
    ("F16", 2, 18, 0, 8, 64, 1),        # nope not a multiple of 4: the register-block absorb
])
def test_projections_ragged_shapes(gpu, fmt, heads, nope, rope, vdim, kv_lora, nq):
    qt, want_qt, out, want_out = run_proj(fmt, heads, nope, rope, vdim, kv_lora, nq, seed=nope + vdim)
    assert_exact(qt, want_qt, f"{fmt} absorb")
    assert_exact(out, want_out, f"{fmt} W_UV")


def test_zero_queries_and_errors(gpu):
    raw, _ = kvb_rows("BF16", 2, 4, 4, 64, 1)
    kvb = dev(raw.reshape(-1))
    empty = torch.empty(0, dtype=torch.float32, device="cuda")
    qr.mla_q_absorb_dev(kvb, 2, 2, 4, 0, 4, 64, empty, empty)
    q = dev(normal(1, (2, 4)))
    qt = torch.empty((2, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(qr.QrInvalidArgument):
        qr.mla_q_absorb_dev(kvb, 5, 2, 4, 0, 4, 64, q, qt)          # Q2_K is not decoded here
    with pytest.raises(qr.QrInvalidArgument):
        qr.mla_q_absorb_dev(kvb, 2, 2, 4, 0, 4, 60, q, qt)          # kv_lora not a multiple of 8
    with pytest.raises(qr.QrInvalidArgument):
        qr.mla_q_absorb_dev(kvb, 4, 2, 4, 0, 4, 48, q, qt)          # Q8_0 needs 32-weight blocks
    padded = dev(np.concatenate([raw.reshape(-1), np.zeros(2, np.uint8)]))
    with pytest.raises(qr.QrInvalidArgument):
        qr.mla_wuv_dev(padded[2:], 2, 2, 4, 4, 64, dev(normal(2, (2, 64))), qt)  # misaligned kvb
    with pytest.raises(ValueError):
        qr.mla_wuv_dev(kvb, 2, 2, 4, 4, 64, dev(normal(2, (2, 64))), qt[:1, :3])  # output too short


def _layer_inputs(heads, nope, rope, vdim, kv_lora, n, dtype, fmt, seed):
    lat = normal(seed, (n, kv_lora + rope))
    bits, latd = to_dtype_bits(lat, dtype)
    raw, w = kvb_rows(fmt, heads, nope, vdim, kv_lora, seed + 1)
    q = normal(seed + 2, (heads, nope + rope))
    return bits, latd, raw, w, q


def _layer_oracle(latd, w, q, heads, nope, rope, vdim, kv_lora, pos):
    qt = oracle.mla_q_absorb(q, w, heads, nope, rope, vdim, kv_lora)
    qrp = q[:, nope:]
    s = np.float32(1.0) / np.sqrt(np.float32(nope + rope))
    u = oracle.mla_attention(latd[:pos + 1], qt, qrp, kv_lora, rope, float(s))
    return oracle.mla_wuv(u, w, heads, nope, vdim, kv_lora)


@pytest.mark.parametrize("dtype,fmt,heads,rope,n,pos", [
    ("bf16", "BF16", 128, 64, 4096, None),   # C5 layer shape at 4K positions
    ("f16", "Q8_0", 32, 64, 1000, 700),
    ("bf16", "Q4_K", 16, 0, 600, None),      # NoPE
    ("f32", "Q6_K", 8, 64, 300, None),       # generic fp32 attention kernel
])
def test_attend_absorbed_layer(gpu, dtype, fmt, heads, rope, n, pos):
    """qr_mla_attend_absorbed = W_UV(attention(absorb(q))) for one token; host and device forms."""
    nope, vdim, kv_lora = 128, 128, 512
    bits, latd, raw, w, q = _layer_inputs(heads, nope, rope, vdim, kv_lora, n, dtype, fmt, seed=n + heads)
    p = n - 1 if pos is None else pos
    want = _layer_oracle(latd, w, q, heads, nope, rope, vdim, kv_lora, p)
    code = quant.FMT[fmt]
    tol = 1e-4 if dtype == "f32" else 5e-3
    with qr.MlaLatentCache(1, kv_lora + rope, n, dtype=dtype, rope=rope) as m:
        m.AppendRange(0, 0, bits, src_dtype=dtype)
        W = qr.Weight(code, heads * (nope + vdim), kv_lora, raw)
        got = m.AttendAbsorbed(0, p, q, W, nope, vdim)
        a, r = assert_close(got, want, 1e-3, tol, f"{dtype}/{fmt} host")
        out = torch.empty((heads, vdim), dtype=torch.float32, device="cuda")
        m.AttendAbsorbedDev(0, p, dev(q), W, code, nope, vdim, out)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), got), "device and host forms differ"
        W.close()
    print(f"{dtype}/{fmt} H{heads}: vs oracle max-abs {a:.2e} rel {r:.2e}")


def test_attend_absorbed_equals_expanded(gpu):
    """Cli/Commands.cs:2065-2152 through the fused call: the absorbed layer block equals the
    expanded-K/V attention in fp64 (H4, kvLora 8, nope 4, v 4, rope 16, seq 10)."""
    heads, kv_lora, nope, vdim, rope, seq = 4, 8, 4, 4, 16, 10
    rng = np.random.default_rng(31)
    R = lambda *s: (rng.random(s) * 2 - 1).astype(np.float32)  # noqa: E731
    q, kvb, lat = R(heads, nope + rope), R(heads * (nope + vdim), kv_lora), R(seq, kv_lora + rope)
    scale = 1 / math.sqrt(nope + rope)
    with qr.MlaLatentCache(1, kv_lora + rope, 64, rope=rope) as m:
        m.AppendRange(0, 0, lat)
        W = qr.Weight("F32", heads * (nope + vdim), kv_lora, kvb.view(np.uint8))
        got = m.AttendAbsorbed(0, seq - 1, q, W, nope, vdim)
        W.close()
    want = oracle.mla_expanded_f64(q, kvb, lat, heads, nope, rope, vdim, kv_lora, scale)
    assert np.max(np.abs(got - want)) <= 1e-4, errors(got, want)


def test_attend_absorbed_errors(gpu):
    kv_lora, rope = 64, 16
    with qr.MlaLatentCache(1, kv_lora + rope, 300, rope=rope) as m:
        m.AppendRange(0, 0, normal(3, (10, kv_lora + rope)))
        raw, _ = kvb_rows("F16", 4, 8, 8, kv_lora, 2)
        W = qr.Weight("F16", 4 * 16, kv_lora, raw)
        q = normal(4, (4, 8 + rope))
        with pytest.raises(qr.QrInvalidArgument):
            m.AttendAbsorbed(0, 9, q, W, 8, 4)        # kvb rows do not match heads*(nope+vdim)
        with pytest.raises(qr.QrNotResident):
            m.AttendAbsorbed(0, 260, q, W, 8, 8)      # page of position 260 never appended
        with pytest.raises(qr.QrInvalidArgument):
            qr.Weight("Q8_0", 4, 48, np.zeros(4 * 51, np.uint8))  # 48 weights are not whole blocks
        W.close()
