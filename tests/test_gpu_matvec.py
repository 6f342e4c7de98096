"""GPU parity of the fused dequant + dot MatVec (DotKernels.MatVec, DotKernels.cs:599-633).

Bar: bit-exact.  Each row follows its format's DotRow operation order
(DotKernels.cs:24-447: the 8-lane Vector256 sums of the fp formats with the vector
half converter, Q8_0/Q4_0 per-block lanes, Q4_K sub-block terms, Q6_K's 256-term
chains, blocks added in order), so y must equal the oracle exactly.
"""
import numpy as np
import pytest
import torch

import qauntrunner_amd as qr
from oracle import oracle
from tests import quant
from tests.util import normal

pytestmark = pytest.mark.gpu

FORMATS = ["F32", "F16", "BF16", "Q4_0", "Q8_0", "Q4_K", "Q6_K"]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def run(fmt, rows, cols, nq, seed, std=0.05):
    code = quant.FMT[fmt]
    raw, _ = quant.random_rows(code, rows, cols, seed, std)
    x = normal(seed + 1, (nq, cols))
    y = torch.empty((nq, rows), dtype=torch.float32, device="cuda")
    qr.matvec_dev(dev(raw.reshape(-1)), code, rows, cols, dev(x), y)
    torch.cuda.synchronize()
    want = np.stack([oracle.matvec(code, raw, cols, x[b]) for b in range(nq)])
    return y.cpu().numpy(), want, raw, x


def assert_exact(got, want, what):
    bad = np.flatnonzero(got.reshape(-1) != want.reshape(-1))
    assert bad.size == 0, (f"{what}: {bad.size} of {got.size} differ, first at {bad[0]}: "
                           f"{got.reshape(-1)[bad[0]]!r} vs {want.reshape(-1)[bad[0]]!r}")


@pytest.mark.parametrize("fmt", FORMATS)
def test_matvec_bit_exact_per_format(gpu, fmt):
    """300 rows x 1024 columns, one vector."""
    got, want, _, _ = run(fmt, 300, 1024, 1, seed=quant.FMT[fmt] + 3)
    assert_exact(got, want, fmt)


@pytest.mark.parametrize("fmt", ["F32", "F16", "BF16", "Q8_0", "Q4_K"])
@pytest.mark.parametrize("rows", [(512, 128, 128), (300, 13, 77, 8)])
def test_matvec_group_matches_single_calls(gpu, fmt, rows):
    """qr_matvec_group_dev: the matrices of one x (wq/wk/wv-like, and row counts that are not
    multiples of 8) in one launch give each matrix's single-call y, bit for bit."""
    code, cols, nq = quant.FMT[fmt], 1024, 2
    raws = [quant.random_rows(code, r, cols, 70 + m, 0.05)[0] for m, r in enumerate(rows)]
    x = dev(normal(79, (nq, cols)))
    ws = [dev(raw.reshape(-1)) for raw in raws]
    ys = [torch.full((nq, r), float("nan"), device="cuda") for r in rows]
    qr.matvec_group_dev(ws, code, list(rows), cols, x, ys)
    singles = [torch.empty((nq, r), device="cuda") for r in rows]
    for m, r in enumerate(rows):
        qr.matvec_dev(ws[m], code, r, cols, x, singles[m])
    torch.cuda.synchronize()
    for m in range(len(rows)):
        assert_exact(ys[m].cpu().numpy(), singles[m].cpu().numpy(), f"{fmt} group member {m}")
    want = np.stack([oracle.matvec(code, raws[1], cols, x[b].cpu().numpy()) for b in range(nq)])
    assert_exact(ys[1].cpu().numpy(), want, f"{fmt} group member 1 vs the oracle")


@pytest.mark.parametrize("fmt", ["F16", "Q8_0", "Q4_K"])
def test_matvec_llama_8b_projection(gpu, fmt):
    """The 8B wq / wo shape: 4096 x 4096."""
    got, want, _, _ = run(fmt, 4096, 4096, 1, seed=40)
    assert_exact(got, want, f"{fmt} 4096x4096")


@pytest.mark.parametrize("fmt,rows,cols,nq", [
    ("Q8_0", 64, 14336, 1),     # the FFN down shape's columns: four slabs, the last partial
    ("Q4_K", 40, 14336, 2),
    ("F16", 33, 14336, 1),      # lane sums continue across slabs
    ("Q6_K", 17, 8448, 3),
    ("Q4_0", 5, 4128, 2),       # 129 blocks: one block past a slab
    ("BF16", 1, 8, 1),          # one chunk
    ("F32", 7, 4104, 4),        # two slabs, the second a single chunk
])
def test_matvec_ragged_shapes(gpu, fmt, rows, cols, nq):
    got, want, _, _ = run(fmt, rows, cols, nq, seed=rows + cols)
    assert_exact(got, want, f"{fmt} {rows}x{cols} nq{nq}")


@pytest.mark.parametrize("fmt,rows,cols,nq", [
    ("Q4_K", 24, 32768, 1),     # 512 items a row: the padded copy of x fills 136 KiB of LDS
    ("Q8_0", 20, 20480, 2),     # 320 block pairs: past the ring's 256, the persistent form
    ("Q4_K", 9000, 4096, 1),    # several tiles per workgroup at two rows a thread
])
def test_matvec_long_rows_and_many_tiles(gpu, fmt, rows, cols, nq):
    """Shapes whose workgroups need more than 64 KiB of LDS, or walk several row tiles."""
    got, want, _, _ = run(fmt, rows, cols, nq, seed=rows + cols)
    assert_exact(got, want, f"{fmt} {rows}x{cols} nq{nq}")


def assert_exact_nan(got, want, what):
    """Bit-exact, except that any NaN matches any NaN (payloads are not compared)."""
    g, w = got.reshape(-1), want.reshape(-1)
    bad = np.flatnonzero((g != w) & ~(np.isnan(g) & np.isnan(w)))
    assert bad.size == 0, f"{what}: {bad.size} of {g.size} differ, first at {bad[0]}: {g[bad[0]]!r} vs {w[bad[0]]!r}"


@pytest.mark.parametrize("fmt", FORMATS)
def test_matvec_extreme_inputs(gpu, fmt):
    """Vector 0 holds finite values at and above 2^103 (1.2e31, -3.0e38): the Q4_K kernel,
    which otherwise takes its products from x prescaled by 2^24, falls back to unscaled x
    for that vector's workgroups.  Vector 1 holds subnormals, tiny values and signed zeros;
    vector 2 an infinity and a NaN.  Every row must still equal the oracle."""
    rows, cols = 96, 4096
    code = quant.FMT[fmt]
    raw, _ = quant.random_rows(code, rows, cols, 60 + code, 0.05)
    x = normal(61, (3, cols))
    x[0, [5, 700, 4000]] = [np.float32(1.2e31), np.float32(-3.0e38), np.float32(2.0 ** 103)]
    x[1, [0, 1, 2, 3, 33, 64, 300]] = [1e-40, -1e-45, 0.0, -0.0, 1e-38, -2e-39, 5e-30]
    x[2, [17, 2049]] = [np.inf, np.nan]
    y = torch.empty((3, rows), dtype=torch.float32, device="cuda")
    qr.matvec_dev(dev(raw.reshape(-1)), code, rows, cols, dev(x), y)
    torch.cuda.synchronize()
    with np.errstate(all="ignore"):
        want = np.stack([oracle.matvec(code, raw, cols, x[b]) for b in range(3)])
    got = y.cpu().numpy()
    for b in range(3):
        assert_exact_nan(got[b], want[b], f"{fmt} vector {b}")
    assert np.any(~np.isfinite(want[0])) or np.all(np.abs(want[0]) > 1e20)


def test_matvec_f16_exponent_31_like_the_reference(gpu):
    """Halves with exponent 31 decode as finite 2^16-scale values in DotF16's vector path."""
    rows, cols = 4, 64
    w = (np.random.default_rng(2).standard_normal((rows, cols)) * 0.1).astype(np.float16).view(np.uint16)
    w[0, 3], w[1, 10], w[2, 63], w[3, 0] = 0x7C00, 0xFC00, 0x7E01, 0x7BFF
    x = normal(5, (1, cols))
    y = torch.empty((1, rows), dtype=torch.float32, device="cuda")
    qr.matvec_dev(dev(w.view(np.uint8).reshape(-1)), 1, rows, cols, dev(x), y)
    torch.cuda.synchronize()
    want = oracle.matvec(1, w.view(np.uint8), cols, x[0])
    assert np.all(np.isfinite(want))
    assert_exact(y.cpu().numpy()[0], want, "F16 exponent 31")


def test_matvec_host_weight_and_errors(gpu):
    raw, _ = quant.random_rows(quant.FMT["Q8_0"], 96, 512, 9)
    x = normal(10, (3, 512))
    W = qr.Weight("Q8_0", 96, 512, raw)
    got = W.MatVec(x)
    assert_exact(got, np.stack([oracle.matvec(4, raw, 512, x[b]) for b in range(3)]), "host MatVec")
    assert_exact(W.MatVec(x[0]), oracle.matvec(4, raw, 512, x[0]), "host MatVec, one vector")
    yw = torch.empty((3, 192), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="Weight is format"):
        qr.matvec_dev(W, 4, 192, 512, dev(x), yw)          # more rows than the Weight holds
    with pytest.raises(ValueError, match="Weight is format"):
        qr.matvec_dev(W, 6, 96, 512, dev(x), yw)           # another format
    W.close()
    buf = dev(raw.reshape(-1))
    y = torch.empty((1, 96), dtype=torch.float32, device="cuda")
    xs = dev(x[:1])
    with pytest.raises(qr.QrInvalidArgument):
        qr.matvec_dev(buf, 5, 96, 512, xs, y)             # Q2_K is not decoded here
    with pytest.raises(qr.QrInvalidArgument):
        qr.matvec_dev(buf, 4, 96, 500, xs, y)             # not whole Q8_0 blocks
    padded = dev(np.concatenate([raw.reshape(-1), np.zeros(2, np.uint8)]))
    with pytest.raises(qr.QrInvalidArgument):
        qr.matvec_dev(padded[2:], 4, 96, 512, xs, y)      # misaligned weights (all rows inside the buffer)
    with pytest.raises(qr.QrInvalidArgument):
        qr.matvec_dev(buf, 1, 8, 12, dev(np.zeros(12, np.float32)), y)   # F16 cols not a multiple of 8
    qr.matvec_dev(buf, 4, 0, 512, xs, y)                  # zero rows: nothing to do
