"""GPU tests of the device-position decode step: qr_kv_append_rope_step_dev (Ensure + RoPE +
Append of StreamingEngine.cs:245-248 with PagedKvCache.Ensure, PagedKvCache.cs:41-60, on the
device) and qr_kv_attention_step_dev (PagedKvCache.Attention, :83-136, with the position read on
the device).

Both are checked against the host-position path on a second cache fed the same rows:
* stored K/V rows and the rotated q are bit-identical (the same kernels at the same positions);
* attention agrees within 2e-6 of max|out| (fp32 caches) or 1e-5 (fp16 caches): the device
  path plans its splits for max_seq, the host path for the actual length, so the split merge
  sums in another order;
* SeqLen, BytesUsed and the page accounting agree once the host reads the device state back,
  and host-path appends after device steps continue on fresh pages.
The graph test captures one step (append + attention, two layers) in a HIP graph, replays it at
advancing positions across page boundaries with eager updates of the position and the rows in
between, and checks every replay against the host path.
"""
import numpy as np
import pytest

import qauntrunner_amd as qr
from qauntrunner_amd._lib import QrOutOfMemory, QrOutOfRange
from tests.util import errors, normal

pytestmark = pytest.mark.gpu

THETA = 500000.0


def _rows(seed, n, heads, kv_heads, D):
    return (normal(seed, (n, heads * D)), normal(seed + 1, (n, kv_heads * D)), normal(seed + 2, (n, kv_heads * D)))


def _host_step(torch, kv, layer, pos, q, k, v, out):
    """Host-position reference step: rotates q in place, appends k/v, attends 0..pos."""
    kv.AppendRopeDev(layer, pos, q, k, v, THETA)
    kv.AttentionDev(layer, [0], [pos], q, out, 1.0 / np.sqrt(kv.HeadDim))


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_device_steps_match_the_host_path(gpu, dtype):
    import torch

    heads, kv_heads, D, max_seq = 8, 2, 128, 2048
    p0, steps = 250, 20  # crosses the page boundary at 256
    Q, K, V = _rows(700, p0 + steps, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, max_seq, kv_dtype=dtype) as A, \
            qr.PagedKvCache(1, heads, kv_heads, D, max_seq, kv_dtype=dtype) as B:
        # a prefix through the host path on both caches
        for kv in (A, B):
            kv.AppendRopeDev(0, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        pos_dev = torch.zeros(1, dtype=torch.int32, device=gpu)
        for t in range(p0, p0 + steps):
            qa, qb = dev(Q[t]), dev(Q[t])
            oa = torch.empty(heads * D, device=gpu)
            ob = torch.empty(heads * D, device=gpu)
            _host_step(torch, A, 0, t, qa, dev(K[t]), dev(V[t]), oa)
            pos_dev.fill_(t)
            B.AppendRopeStepDev(0, pos_dev, qb, dev(K[t]), dev(V[t]), THETA)
            B.AttentionStepDev(0, [0], pos_dev, qb, ob, scale)
            torch.cuda.synchronize()
            assert torch.equal(qa, qb), f"rotated q differs at {t}"
            want, got = oa.cpu().numpy(), ob.cpu().numpy()
            tol = (2e-6 if dtype == "f32" else 1e-5) * float(np.max(np.abs(want)))
            assert float(np.max(np.abs(got - want))) <= tol, f"attention at {t}"
        # the host reads the device accounting back
        assert B.SeqLen == A.SeqLen == p0 + steps
        assert B.BytesUsed == A.BytesUsed
        ka, va = A.Read(0, 0, p0 + steps)
        kb, vb = B.Read(0, 0, p0 + steps)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        # host-path appends continue after device steps
        t = p0 + steps
        for kv in (A, B):
            kv.AppendRopeDev(0, t, dev(Q[t - 1]), dev(K[t - 1]), dev(V[t - 1]), THETA)
        assert B.SeqLen == A.SeqLen == t + 1 and B.BytesUsed == A.BytesUsed
        ka, va = A.Read(0, t, 1)
        kb, vb = B.Read(0, t, 1)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)
        # Reset / Truncate reach the device copy: the next device step sees SeqLen from there
        B.Truncate(100)
        assert B.SeqLen == 100
        pos_dev.fill_(100)
        B.AppendRopeStepDev(0, pos_dev, dev(Q[0]), dev(K[0]), dev(V[0]), THETA)
        assert B.SeqLen == 101


def test_device_step_reports_a_full_pool_and_a_bad_position(gpu):
    import torch

    heads, kv_heads, D = 4, 2, 64
    with qr.PagedKvCache(1, heads, kv_heads, D, 100000) as kv:
        kv.Reserve(16)  # 16 pages: positions up to 4095
        pos = torch.tensor([4000], dtype=torch.int32, device=gpu)
        k = torch.ones(kv_heads * D, device=gpu)
        kv.AppendRopeStepDev(0, pos, None, k, k, THETA)
        assert kv.SeqLen == 4001
        pos.fill_(5000)  # needs page 19: the pool holds 16
        kv.AppendRopeStepDev(0, pos, None, k, k, THETA)
        with pytest.raises(QrOutOfMemory):
            kv.SeqLen
        assert kv.SeqLen == 4001  # reported once; the append was skipped
        pos.fill_(100000)  # outside [0, max_seq)
        kv.AppendRopeStepDev(0, pos, None, k, k, THETA)
        with pytest.raises(QrOutOfRange):
            kv.SeqLen
        assert kv.SeqLen == 4001


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_captured_decode_step_replays_at_advancing_positions(gpu, dtype):
    import torch

    heads, kv_heads, D, max_seq, layers = 8, 2, 128, 4096, 2
    p0, steps = 500, 24  # crosses the page boundary at 512
    Q, K, V = _rows(800, p0 + steps + 1, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(layers, heads, kv_heads, D, max_seq, kv_dtype=dtype) as A, \
            qr.PagedKvCache(layers, heads, kv_heads, D, max_seq, kv_dtype=dtype) as B:
        for kv in (A, B):
            for layer in range(layers):
                kv.AppendRopeDev(layer, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        B.Reserve(64)  # the pool cannot grow inside a capture
        pos_dev = torch.zeros(1, dtype=torch.int32, device=gpu)
        qbuf = [torch.empty(heads * D, device=gpu) for _ in range(layers)]
        kbuf, vbuf = torch.empty(kv_heads * D, device=gpu), torch.empty(kv_heads * D, device=gpu)
        obuf = [torch.empty(heads * D, device=gpu) for _ in range(layers)]

        def step_b(stream=None):
            for layer in range(layers):
                B.AppendRopeStepDev(layer, pos_dev, qbuf[layer], kbuf, vbuf, THETA, stream=stream)
                B.AttentionStepDev(layer, [0], pos_dev, qbuf[layer], obuf[layer], scale, stream=stream)

        def load(t):
            pos_dev.fill_(t)
            kbuf.copy_(dev(K[t]))
            vbuf.copy_(dev(V[t]))
            for layer in range(layers):
                qbuf[layer].copy_(dev(Q[t]))

        def check(t):
            for layer in range(layers):
                qa, oa = dev(Q[t]), torch.empty(heads * D, device=gpu)
                _host_step(torch, A, layer, t, qa, dev(K[t]), dev(V[t]), oa)
                torch.cuda.synchronize()
                assert torch.equal(qa, qbuf[layer]), f"rotated q, layer {layer}, position {t}"
                want, got = oa.cpu().numpy(), obuf[layer].cpu().numpy()
                tol = (2e-6 if dtype == "f32" else 1e-5) * float(np.max(np.abs(want)))
                assert float(np.max(np.abs(got - want))) <= tol, f"attention, layer {layer}, position {t}"

        # the cache's first device-side step runs eagerly (it also sizes the split workspace)
        load(p0)
        step_b()
        torch.cuda.synchronize()
        check(p0)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            load(p0 + 1)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            step_b()
        # capture does not run the work: replay every position, eager updates in between
        for t in range(p0 + 1, p0 + steps + 1):
            load(t)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            check(t)
        assert B.SeqLen == A.SeqLen == p0 + steps + 1
        assert B.BytesUsed == A.BytesUsed
        for layer in range(layers):
            ka, va = A.Read(layer, 0, p0 + steps + 1)
            kb, vb = B.Read(layer, 0, p0 + steps + 1)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {layer}"


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_decode_step_spreads_short_sequences_over_the_planned_splits(gpu, dtype):
    """max_seq 131072 bounds the plan (many splits); entries at 3,000 and 9,000 positions
    spread over them on the device and agree with the host-planned call."""
    import torch

    heads, kv_heads, D, max_seq = 8, 2, 128, 131072
    n = 9001
    Q, K, V = _rows(900, n, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, max_seq, kv_dtype=dtype, max_batch=2) as kv:
        for s in range(2):
            kv.AppendRangeDev(0, 0, dev(K), dev(V), seq_id=s)
        ids, pos = [0, 1], [2999, 9000]
        q = dev(Q[:2])
        want = torch.empty_like(q)
        kv.AttentionDev(0, ids, pos, q, want, scale)
        got = torch.empty_like(q)
        kv.AttentionStepDev(0, ids, torch.tensor(pos, dtype=torch.int32, device=gpu), q, got, scale)
        torch.cuda.synchronize()
        w, g = want.cpu().numpy(), got.cpu().numpy()
        tol = (2e-6 if dtype == "f32" else 1e-5) * float(np.max(np.abs(w)))
        assert float(np.max(np.abs(g - w))) <= tol


def _chunk_host_step(kv, layer, p0, q, k, v, out):
    """Host-position reference: rotates q in place, appends k/v, causal attention of the chunk."""
    kv.AppendRopeDev(layer, p0, q, k, v, THETA)
    kv.AttentionChunkDev(layer, p0, q, out, 1.0 / np.sqrt(kv.HeadDim))


@pytest.mark.parametrize("dtype,max_seq", [("f16", 4096), ("f16", 65536), ("f32", 4096)])
def test_chunk_steps_match_the_host_path(gpu, dtype, max_seq):
    """qr_kv_append_rope_chunk_step_dev + qr_kv_attention_chunk_step_dev against the host-
    position chunk calls: 16-bit caches take the MFMA chunk kernel (its keys spread over the
    splits planned for max_seq), fp32 caches one decode entry per query."""
    import torch

    heads, kv_heads, D = 8, 2, 128
    p0, nq = 250, 12  # the chunk crosses the page boundary at 256
    Q, K, V = _rows(1000, p0 + 2 * nq, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    with qr.PagedKvCache(1, heads, kv_heads, D, max_seq, kv_dtype=dtype) as A, \
            qr.PagedKvCache(1, heads, kv_heads, D, max_seq, kv_dtype=dtype) as B:
        for kv in (A, B):
            kv.AppendRopeDev(0, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        pos0 = torch.zeros(1, dtype=torch.int32, device=gpu)
        for c in range(2):
            t = p0 + c * nq
            qa, qb = dev(Q[t:t + nq]), dev(Q[t:t + nq])
            oa, ob = torch.empty_like(qa), torch.empty_like(qb)
            _chunk_host_step(A, 0, t, qa, dev(K[t:t + nq]), dev(V[t:t + nq]), oa)
            pos0.fill_(t)
            B.AppendRopeChunkStepDev(0, pos0, qb, dev(K[t:t + nq]), dev(V[t:t + nq]), THETA)
            B.AttentionChunkStepDev(0, pos0, qb, ob, 1.0 / np.sqrt(D))
            torch.cuda.synchronize()
            assert torch.equal(qa, qb), f"rotated q, chunk {c}"
            w, g = oa.cpu().numpy(), ob.cpu().numpy()
            tol = (2e-6 if dtype == "f32" else 1e-5) * float(np.max(np.abs(w)))
            assert float(np.max(np.abs(g - w))) <= tol, f"attention, chunk {c}"
        assert B.SeqLen == A.SeqLen == p0 + 2 * nq
        assert B.BytesUsed == A.BytesUsed
        ka, va = A.Read(0, 0, p0 + 2 * nq)
        kb, vb = B.Read(0, 0, p0 + 2 * nq)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_captured_chunk_step_replays_at_advancing_positions(gpu, dtype):
    """A verify-sized step (8 draft queries, append + attention, two layers) captured once
    and replayed at advancing chunk positions across a page boundary."""
    import torch

    heads, kv_heads, D, max_seq, layers, nq = 8, 2, 128, 8192, 2, 8
    p0, chunks = 480, 6  # 480 + 48 crosses 512
    Q, K, V = _rows(1100, p0 + nq * (chunks + 1), heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(layers, heads, kv_heads, D, max_seq, kv_dtype=dtype) as A, \
            qr.PagedKvCache(layers, heads, kv_heads, D, max_seq, kv_dtype=dtype) as B:
        for kv in (A, B):
            for layer in range(layers):
                kv.AppendRopeDev(layer, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        B.Reserve(64)
        pos0 = torch.zeros(1, dtype=torch.int32, device=gpu)
        qbuf = [torch.empty(nq, heads * D, device=gpu) for _ in range(layers)]
        kbuf, vbuf = torch.empty(nq, kv_heads * D, device=gpu), torch.empty(nq, kv_heads * D, device=gpu)
        obuf = [torch.empty(nq, heads * D, device=gpu) for _ in range(layers)]

        def step_b():
            for layer in range(layers):
                B.AppendRopeChunkStepDev(layer, pos0, qbuf[layer], kbuf, vbuf, THETA)
                B.AttentionChunkStepDev(layer, pos0, qbuf[layer], obuf[layer], scale)

        def load(t):
            pos0.fill_(t)
            kbuf.copy_(dev(K[t:t + nq]))
            vbuf.copy_(dev(V[t:t + nq]))
            for layer in range(layers):
                qbuf[layer].copy_(dev(Q[t:t + nq]))

        def check(t):
            for layer in range(layers):
                qa, oa = dev(Q[t:t + nq]), torch.empty(nq, heads * D, device=gpu)
                _chunk_host_step(A, layer, t, qa, dev(K[t:t + nq]), dev(V[t:t + nq]), oa)
                torch.cuda.synchronize()
                assert torch.equal(qa, qbuf[layer]), f"rotated q, layer {layer}, chunk at {t}"
                w, g = oa.cpu().numpy(), obuf[layer].cpu().numpy()
                tol = (2e-6 if dtype == "f32" else 1e-5) * float(np.max(np.abs(w)))
                assert float(np.max(np.abs(g - w))) <= tol, f"attention, layer {layer}, chunk at {t}"

        load(p0)
        step_b()  # eager first call: device accounting and split workspace
        torch.cuda.synchronize()
        check(p0)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            load(p0 + nq)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            step_b()
        for c in range(1, chunks + 1):
            t = p0 + c * nq
            load(t)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            check(t)
        end = p0 + nq * (chunks + 1)
        assert B.SeqLen == A.SeqLen == end
        for layer in range(layers):
            ka, va = A.Read(layer, 0, end)
            kb, vb = B.Read(layer, 0, end)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"layer {layer}"


@pytest.mark.parametrize("dtype,heads,rope,max_seq", [("bf16", 32, 64, 4096), ("bf16", 32, 64, 65536),
                                                      ("f32", 8, 64, 4096)])
def test_mla_steps_match_the_host_path(gpu, dtype, heads, rope, max_seq):
    """qr_mla_append_step_dev + qr_mla_attention_step_dev against the host-position calls:
    16-bit latents take the MFMA tile kernel (the sequence spreads over the splits planned for
    max_seq), fp32 latents the generic kernel; single-row and multi-row appends."""
    import torch

    kv_lora = 512
    W = kv_lora + rope
    p0 = 250
    rows = normal(1200, (p0 + 40, W)).astype(np.float32)
    qt, qr_ = normal(1201, (heads, kv_lora)), normal(1202, (heads, rope))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1 / np.sqrt(192)
    with qr.MlaLatentCache(1, W, max_seq, dtype=dtype, rope=rope) as A, \
            qr.MlaLatentCache(1, W, max_seq, dtype=dtype, rope=rope) as B:
        for m in (A, B):
            m.AppendRangeDev(0, 0, dev(rows[:p0]))
        pos = torch.zeros(1, dtype=torch.int32, device=gpu)
        t = p0
        for n in (1, 1, 5, 1, 12):  # crosses the page boundary at 256
            A.AppendRangeDev(0, t, dev(rows[t:t + n]))
            pos.fill_(t)
            B.AppendStepDev(0, pos, dev(rows[t:t + n]))
            t += n
            ua, ub = torch.empty(heads, kv_lora, device=gpu), torch.empty(heads, kv_lora, device=gpu)
            A.AbsorbedAttentionDev(0, t - 1, dev(qt), dev(qr_), ua, scale)
            pos.fill_(t - 1)
            B.AbsorbedAttentionStepDev(0, pos, dev(qt), dev(qr_), ub, scale)
            torch.cuda.synchronize()
            want, got = ua.cpu().numpy(), ub.cpu().numpy()
            a, r = errors(got, want)
            assert r <= (1e-6 if dtype == "f32" else 1e-3), f"attention at {t - 1}: rel {r:.2e}"
        assert B.SeqLen == A.SeqLen == t
        assert B.BytesUsed == A.BytesUsed and B.PageCount(0) == A.PageCount(0)
        for pg in range(A.PageCount(0)):
            assert np.array_equal(A.Page(0, pg), B.Page(0, pg)), f"page {pg}"
        B.Truncate(100)
        pos.fill_(100)
        B.AppendStepDev(0, pos, dev(rows[:1]))
        assert B.SeqLen == 101


def test_captured_mla_layer_step_replays_at_advancing_positions(gpu):
    """Append + absorbed layer block (q-absorb, attention, W_UV) at a device position,
    captured once and replayed at 20 advancing positions across a page boundary."""
    import torch

    heads, nope, rope, vdim, kv_lora, max_seq = 32, 128, 64, 128, 512, 8192
    W = kv_lora + rope
    p0, steps = 500, 20
    rows = normal(1300, (p0 + steps + 1, W)).astype(np.float32)
    kvb = normal(1301, (heads * (nope + vdim), kv_lora)).astype(np.float32) * 0.05
    qs = normal(1302, (p0 + steps + 1, heads * (nope + rope)))
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    with qr.MlaLatentCache(1, W, max_seq, dtype="bf16", rope=rope) as A, \
            qr.MlaLatentCache(1, W, max_seq, dtype="bf16", rope=rope) as B:
        Wt = qr.Weight("F32", heads * (nope + vdim), kv_lora, kvb.view(np.uint8))
        for m in (A, B):
            m.AppendRangeDev(0, 0, dev(rows[:p0]))
        B.Reserve(16)
        pos = torch.zeros(1, dtype=torch.int32, device=gpu)
        row_buf = torch.empty(1, W, device=gpu)
        q_buf = torch.empty(heads, nope + rope, device=gpu)
        out_b = torch.empty(heads, vdim, device=gpu)

        def step_b():
            B.AppendStepDev(0, pos, row_buf)
            B.AttendAbsorbedStepDev(0, pos, q_buf, Wt, Wt.Fmt, nope, vdim, out_b)

        def load(t):
            pos.fill_(t)
            row_buf.copy_(dev(rows[t:t + 1]))
            q_buf.copy_(dev(qs[t].reshape(heads, nope + rope)))

        def check(t):
            A.AppendRangeDev(0, t, dev(rows[t:t + 1]))
            out_a = torch.empty(heads, vdim, device=gpu)
            A.AttendAbsorbedDev(0, t, dev(qs[t].reshape(heads, nope + rope)), Wt, Wt.Fmt, nope, vdim, out_a)
            torch.cuda.synchronize()
            a, r = errors(out_b.cpu().numpy(), out_a.cpu().numpy())
            assert r <= 1e-3, f"layer block at {t}: rel {r:.2e}"

        load(p0)
        step_b()  # eager first call: device accounting, workspaces
        torch.cuda.synchronize()
        check(p0)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            load(p0 + 1)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            step_b()
        for t in range(p0 + 1, p0 + steps + 1):
            load(t)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            check(t)
        assert B.SeqLen == A.SeqLen == p0 + steps + 1
        for pg in range(A.PageCount(0)):
            assert np.array_equal(A.Page(0, pg), B.Page(0, pg)), f"page {pg}"
        Wt.close()


def test_captured_step_keeps_its_buffers_when_host_calls_grow_them(gpu):
    """A graph captured over device-position steps keeps the pool and workspace addresses it
    was recorded with.  Host calls made between replays that need a larger split workspace
    get a new one while the graph keeps the old allocation; a host append that would grow
    the pool is refused (QrOutOfMemory) instead of moving the pool under the graph.  Every
    replay still matches the host path."""
    import torch

    heads, kv_heads, D, max_seq, seqs = 8, 2, 128, 4096, 16
    p0, steps, other = 500, 6, 2000
    Q, K, V = _rows(1100, p0 + steps + 1, heads, kv_heads, D)
    _, Ko, Vo = _rows(1200, other, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, max_seq) as A, \
            qr.PagedKvCache(1, heads, kv_heads, D, max_seq, max_batch=seqs) as B:
        for kv in (A, B):
            kv.AppendRopeDev(0, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        for s in range(1, seqs):  # the other sequences are filled before the capture
            B.AppendRangeDev(0, 0, dev(Ko), dev(Vo), seq_id=s)
        pos_dev = torch.zeros(1, dtype=torch.int32, device=gpu)
        qb, ob = torch.empty(heads * D, device=gpu), torch.empty(heads * D, device=gpu)
        kb, vb = torch.empty(kv_heads * D, device=gpu), torch.empty(kv_heads * D, device=gpu)

        def load(t):
            pos_dev.fill_(t)
            qb.copy_(dev(Q[t]))
            kb.copy_(dev(K[t]))
            vb.copy_(dev(V[t]))

        def check(t):
            qa, oa = dev(Q[t]), torch.empty(heads * D, device=gpu)
            _host_step(torch, A, 0, t, qa, dev(K[t]), dev(V[t]), oa)
            torch.cuda.synchronize()
            want, got = oa.cpu().numpy(), ob.cpu().numpy()
            assert float(np.max(np.abs(got - want))) <= 2e-6 * float(np.max(np.abs(want))), f"position {t}"

        load(p0)
        B.AppendRopeStepDev(0, pos_dev, qb, kb, vb, THETA)
        B.AttentionStepDev(0, [0], pos_dev, qb, ob, scale)
        torch.cuda.synchronize()
        check(p0)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            B.AppendRopeStepDev(0, pos_dev, qb, kb, vb, THETA, stream=s)
            B.AttentionStepDev(0, [0], pos_dev, qb, ob, scale, stream=s)
        for i, t in enumerate(range(p0 + 1, p0 + steps + 1)):
            if i == 1:
                # 15 sequences of 2000 positions in one call: a larger split workspace
                ids = list(range(1, seqs))
                qo = dev(normal(1300, (len(ids), heads * D)))
                oo = torch.empty_like(qo)
                B.AttentionDev(0, ids, [other - 1] * len(ids), qo, oo, scale)
                torch.cuda.synchronize()
                assert torch.isfinite(oo).all()
            if i == 2:
                # growing the pool would move it under the graph: refused
                with pytest.raises(QrOutOfMemory, match="captured graph"):
                    B.Reserve(100000)
            load(t)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            check(t)
        assert B.SeqLen == p0 + steps + 1


def test_device_rope_step_rejects_wide_rows_before_claiming_pages(gpu):
    """(heads + kv_heads) * head_dim above 16384 dims per position cannot take a device
    position: the call is refused on the host before the page claim is enqueued, so the
    device accounting stays as it was."""
    import torch

    heads, kv_heads, D = 128, 8, 128
    with qr.PagedKvCache(1, heads, kv_heads, D, 4096) as kv:
        pos = torch.tensor([0], dtype=torch.int32, device=gpu)
        q = torch.ones(heads * D, device=gpu)
        k = torch.ones(kv_heads * D, device=gpu)
        with pytest.raises(qr.QrInvalidArgument, match="dims of K and q"):
            kv.AppendRopeStepDev(0, pos, q, k, k, THETA)
        torch.cuda.synchronize()
        assert kv.SeqLen == 0 and kv.BytesUsed == 0
        kv.AppendRopeStepDev(0, pos, None, k, k, THETA)  # K only: 1024 dims
        assert kv.SeqLen == 1


def test_no_alloc_decode_is_captured_after_a_device_step(gpu):
    """qr_kv_attention_dev_noalloc enqueued under capture right after a device-position
    append does not read the device accounting back (that would wait for the device inside
    the capture); its host-side checks use the host accounting.  Replays equal the eager
    call."""
    import torch

    heads, kv_heads, D, p0 = 8, 2, 128, 700
    Q, K, V = _rows(1400, p0 + 2, heads, kv_heads, D)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    scale = 1.0 / np.sqrt(D)
    with qr.PagedKvCache(1, heads, kv_heads, D, 4096) as kv:
        kv.AppendRopeDev(0, 0, dev(Q[:p0]), dev(K[:p0]), dev(V[:p0]), THETA)
        kv.Reserve(16)
        pos_dev = torch.tensor([p0], dtype=torch.int32, device=gpu)
        qs = dev(Q[p0])
        kv.AppendRopeStepDev(0, pos_dev, qs, dev(K[p0]), dev(V[p0]), THETA)  # the device is now ahead
        q = dev(Q[p0 - 1])
        out = torch.empty(heads * D, device=gpu)
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s):
            kv.AttentionDevNoAlloc(0, [0], [p0 - 1], q, out, scale, stream=s)
        want = torch.empty_like(out)
        kv.AttentionDev(0, [0], [p0 - 1], q, want, scale)  # eager, after a read-back
        for _ in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want)
        assert kv.SeqLen == p0 + 1
