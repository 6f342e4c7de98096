"""The no-allocation decode entry point (qr_kv_attention_dev_noalloc) against the
allocating one (qr_kv_attention_dev): the same kernels and split plan, only the split
partials live in the library's fixed device array, so the outputs must be identical.
Two calls in a row, the second with a smaller input, then a call whose partials would
not fit the array (rejected before any launch)."""
import math

import numpy as np
import pytest

import qauntrunner_amd as qr
from tests.util import to_dtype_bits, normal

pytestmark = pytest.mark.gpu


def _run(kv, gpu, layer, ids, pos, q, scale, noalloc):
    import torch

    qd = torch.from_numpy(q).to(gpu)
    out = torch.full_like(qd, float("nan"))
    (kv.AttentionDevNoAlloc if noalloc else kv.AttentionDev)(layer, ids, pos, qd, out, scale)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_noalloc_decode_matches_the_allocating_call(gpu, dtype):
    heads, kv_heads, D, n = 32, 8, 128, 8192
    scale = 1 / math.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype=dtype, max_batch=4) as kv:
        for s in range(4):
            Kb, _ = to_dtype_bits(normal(1000 + s, (n, kv_heads * D)), dtype)
            Vb, _ = to_dtype_bits(normal(1010 + s, (n, kv_heads * D)), dtype)
            kv.AppendRange(0, 0, Kb, Vb, src_dtype=dtype, seq_id=s)
        # first call: 4 entries over 8192 positions (several splits each)
        ids, pos = [0, 1, 2, 3], [n - 1, n - 1, 5000, 777]
        q = normal(1020, (4, heads * D))
        assert kv.DecodePlan(0, ids, pos)[1] > 1
        want = _run(kv, gpu, 0, ids, pos, q, scale, noalloc=False)
        got = _run(kv, gpu, 0, ids, pos, q, scale, noalloc=True)
        assert np.isfinite(got).all() and np.array_equal(got, want)
        # second call, smaller: one entry over 3000 positions
        ids, pos = [2], [2999]
        q = normal(1021, (1, heads * D))
        want = _run(kv, gpu, 0, ids, pos, q, scale, noalloc=False)
        got = _run(kv, gpu, 0, ids, pos, q, scale, noalloc=True)
        assert np.isfinite(got).all() and np.array_equal(got, want)


def test_noalloc_decode_rejects_partials_beyond_its_array(gpu):
    """64 entries x 128 heads x 2 splits x 520 bytes = 8.5 MB > 8 MiB - 64 KiB: rejected."""
    import torch

    heads, kv_heads, D, n = 128, 1, 128, 8192
    with qr.PagedKvCache(1, heads, kv_heads, D, n, kv_dtype="f16") as kv:
        kv.AppendRange(0, 0, np.zeros((n, D), np.uint16), np.zeros((n, D), np.uint16), src_dtype="f16")
        ids, pos = [0] * 64, [n - 1] * 64
        assert kv.DecodePlan(0, ids, pos) == (16 * 256, 2)
        q = torch.zeros(64, heads * D, device=gpu)
        out = torch.zeros_like(q)
        with pytest.raises(qr.QrOutOfRange):
            kv.AttentionDevNoAlloc(0, ids, pos, q, out, 0.1)
        with pytest.raises(qr.QrInvalidArgument):  # more than 64 entries per call
            kv.AttentionDevNoAlloc(0, [0] * 65, [n - 1] * 65, torch.zeros(65, heads * D, device=gpu),
                                   torch.zeros(65, heads * D, device=gpu), 0.1)
        # the allocating entry point takes the same call
        kv.AttentionDev(0, ids, pos, q, out, 0.1)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
