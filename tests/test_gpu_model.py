"""GPU parity of the .qw -> HBM weight path (ModelStore + PrefetchPipeline, MI355X side).

The reference's own check is "prefetch ON == prefetch OFF logits" (tests/QuantRunner.Tests/
Program.cs:402-422): staging must not change a single result.  Here every weight a layer
loop acquires feeds the bit-exact MatVec, and each output must equal the oracle's DotRow
over the file's bytes, with the pipeline off (tensors served one by one), staging through
the two HBM slots, or every tensor resident.  The loops queue all layers without a host
synchronisation, so a slot overwritten while an earlier layer still reads it would show
as a wrong row.  Bar: bit-exact.
"""
import re

import numpy as np
import pytest
import torch

import qauntrunner_amd as qr
from oracle import oracle
from qauntrunner_amd.store import ModelStoreBuilder
from tests import qwmodel, quant
from tests.util import normal

pytestmark = pytest.mark.gpu

NQ = 2


def inputs(tensors, seed=7):
    cols = sorted({dims[-1] for _, dims, _ in tensors.values()})
    return {c: normal(seed + c, (NQ, c)) for c in cols}


def expected(tensors, xs, names):
    out = {}
    for n in names:
        code, dims, raw = tensors[n]
        out[n] = np.stack([oracle.matvec(code, raw, dims[-1], xs[dims[-1]][b]) for b in range(NQ)])
    return out


def layer_names(tensors, l):
    return [n for n in tensors if n.startswith(f"l{l}.")]


def run_loop(store, pipe, tensors, layers, xs, release=True, streams=None):
    """StreamingEngine's order (StreamingEngine.cs:225-266): Begin(0), then per layer the
    acquires and launches, then Begin(l + 1); everything queued, one synchronisation."""
    xd = {c: torch.from_numpy(v).cuda() for c, v in xs.items()}
    streams = streams or [torch.cuda.current_stream()]
    outs = {}
    if pipe:
        pipe.Begin(0)
    for l in range(layers):
        for i, n in enumerate(layer_names(tensors, l)):
            st = streams[i % len(streams)]
            code, dims, _ = tensors[n]
            rows = int(np.prod(dims[:-1])) if len(dims) > 1 else 1
            w = pipe.Acquire(n, l, st) if pipe else None
            y = torch.empty((NQ, rows), dtype=torch.float32, device="cuda")
            with torch.cuda.stream(st):
                y.record_stream(st)
                qr.matvec_dev(w, code, rows, dims[-1], xd[dims[-1]], y, stream=st)
            outs[n] = y
        if pipe and release:
            for st in streams:
                pipe.Release(l, st)
        if pipe and l + 1 < layers:
            pipe.Begin(l + 1)
    for n in [n for n in tensors if not re.match(r"l\d+\.", n)]:   # tok_emb, final_norm, lm_head
        code, dims, _ = tensors[n]
        rows = dims[0] if len(dims) > 1 else 1
        w = pipe.Acquire(n, -1)
        y = torch.empty((NQ, rows), dtype=torch.float32, device="cuda")
        qr.matvec_dev(w, code, rows, dims[-1], xd[dims[-1]], y)
        outs[n] = y
    torch.cuda.synchronize()
    return {n: v.cpu().numpy() for n, v in outs.items()}


def assert_exact(got, want):
    for n, w in want.items():
        g = got[n]
        bad = np.flatnonzero(g.reshape(-1) != w.reshape(-1))
        assert bad.size == 0, f"{n}: {bad.size} of {g.size} differ, first {g.reshape(-1)[bad[0]]!r} vs " \
                              f"{w.reshape(-1)[bad[0]]!r}"


@pytest.mark.parametrize("fmt", ["Q4_K", "Q8_0", "F16"])
def test_prefetch_on_off_and_resident_match_the_oracle(gpu, tmp_path, fmt):
    path = str(tmp_path / "m.qw")
    layers = 3
    tensors = qwmodel.write(path, layers=layers, fmt=fmt, seed=8)
    xs = inputs(tensors)
    want = expected(tensors, xs, list(tensors))
    results = {}
    for mode in ("off", "staged", "resident"):
        with qr.ModelStore.Open(path) as s:
            pipe = qr.PrefetchPipeline(s, 0 if mode == "off" else 4 << 20)
            if mode == "resident":
                s.MakeResident()
            got = run_loop(s, pipe, tensors, layers, xs)
            assert_exact(got, want)
            results[mode] = got
            if mode == "staged":
                assert pipe.StagedLayers == layers and pipe.SkippedLayers == 0
                assert pipe.BytesStreamed == sum(qwmodel.layer_bytes(tensors, l) for l in range(layers))
                assert pipe.ReadMs > 0
            if mode == "off":
                assert pipe.BytesStreamed == 0 and pipe.StagedLayers == 0
            if mode == "resident":
                assert pipe.BytesStreamed == sum(t[2].size for t in tensors.values())
    for n in tensors:
        assert np.array_equal(results["off"][n], results["staged"][n])


def test_layers_over_budget_fall_back(gpu, tmp_path):
    """PrefetchPipeline.cs:131-135: a layer above the budget is counted and served unstaged."""
    path = str(tmp_path / "moe.qw")
    layers = 3
    tensors = qwmodel.write(path, layers=layers, experts=3, fmt="Q8_0", seed=9)
    xs = inputs(tensors)
    want = expected(tensors, xs, list(tensors))
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, qwmodel.layer_bytes(tensors, 0) - 1)
        assert_exact(run_loop(s, pipe, tensors, layers, xs), want)
        assert (pipe.StagedLayers, pipe.SkippedLayers, pipe.BytesStreamed) == (0, layers, 0)
    with qr.ModelStore.Open(path) as s:   # exactly at the budget: staged (total > budget skips)
        pipe = qr.PrefetchPipeline(s, qwmodel.layer_bytes(tensors, 0))
        assert_exact(run_loop(s, pipe, tensors, layers, xs), want)
        assert (pipe.StagedLayers, pipe.SkippedLayers) == (layers, 0)


@pytest.mark.parametrize("release", [True, False])
def test_many_layers_queued_without_host_sync(gpu, tmp_path, release):
    """Eight layers through two slots: each slot is rewritten three times while earlier
    layers' launches may still be queued.  Without Release, Begin itself fences."""
    path = str(tmp_path / "deep.qw")
    layers = 8
    tensors = qwmodel.write(path, layers=layers, dim=512, ffn=1024, heads=8, fmt="Q8_0", seed=10)
    xs = inputs(tensors)
    want = expected(tensors, xs, list(tensors))
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 64 << 20)
        assert_exact(run_loop(s, pipe, tensors, layers, xs, release=release), want)
        assert pipe.StagedLayers == layers


def test_two_streams_share_a_layer(gpu, tmp_path):
    path = str(tmp_path / "two.qw")
    layers = 4
    tensors = qwmodel.write(path, layers=layers, fmt="Q4_K", seed=11)
    xs = inputs(tensors)
    want = expected(tensors, xs, list(tensors))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 8 << 20)
        assert_exact(run_loop(s, pipe, tensors, layers, xs, streams=streams), want)
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 8 << 20)
        assert_exact(run_loop(s, pipe, tensors, layers, xs, release=False, streams=streams), want)


def test_slots_grow_under_queued_work(gpu, tmp_path):
    """Layers of rising size: each slot reallocates while the other slot's layer is queued."""
    path = str(tmp_path / "grow.qw")
    layers, cols = 6, 512
    b = ModelStoreBuilder(path, {"arch": "llama"})
    tensors = {}
    for i, (name, rows) in enumerate([("lm_head", 64), ("final_norm", 1)] +
                                     [(f"l{l}.wq", 128 * (l + 1)) for l in range(layers)]):
        code = quant.FMT["F32" if name == "final_norm" else "Q4_0"]
        raw, _ = quant.random_rows(code, rows, cols, 50 + i, std=0.02)
        dims = (cols,) if name == "final_norm" else (rows, cols)
        tensors[name] = (code, dims, np.ascontiguousarray(raw).reshape(-1))
        b.Plan(name, dims, code, raw.size)
    b.Commit(lambda n: tensors[n][2])
    xs = inputs(tensors)
    want = expected(tensors, xs, list(tensors))
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 16 << 20)
        assert_exact(run_loop(s, pipe, tensors, layers, xs, release=False), want)
        assert pipe.StagedLayers == layers


def test_begin_minus_one_stages_the_whole_file(gpu, tmp_path):
    """A negative layer takes every tensor but norms and routers (PrefetchPipeline.cs:116-124);
    lm_head is then served from slot 1, norms one by one."""
    path = str(tmp_path / "all.qw")
    tensors = qwmodel.write(path, layers=2, fmt="Q6_K", seed=12)
    xs = inputs(tensors)
    want = expected(tensors, xs, ["lm_head", "final_norm", "l1.wo", "l0.attn_norm"])
    xd = {c: torch.from_numpy(v).cuda() for c, v in xs.items()}
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 32 << 20)
        pipe.Begin(-1)
        pipe.WaitLayer(-1)
        assert pipe.StagedLayers == 1 and pipe.BytesStreamed == qwmodel.layer_bytes(tensors, -1)
        got = {}
        for n in want:
            code, dims, _ = tensors[n]
            rows = dims[0] if len(dims) > 1 else 1
            y = torch.empty((NQ, rows), dtype=torch.float32, device="cuda")
            qr.matvec_dev(pipe.Acquire(n, -1), code, rows, dims[-1], xd[dims[-1]], y)
            got[n] = y
        torch.cuda.synchronize()
        assert_exact({n: v.cpu().numpy() for n, v in got.items()}, want)


def test_acquire_errors(gpu, tmp_path):
    path = str(tmp_path / "e.qw")
    qwmodel.write(path, layers=1, fmt="Q8_0", seed=13)
    with qr.ModelStore.Open(path) as s:
        pipe = qr.PrefetchPipeline(s, 1 << 20)
        with pytest.raises(qr.QrInvalidArgument):
            pipe.Acquire("l0.nope", 0)
        pipe.Begin(0)
        a = pipe.Acquire("l0.wq", 0).data_ptr()
        assert a and a % 256 == 0
        assert pipe.Acquire("l0.wq", 0).data_ptr() == a       # same slot, same address
        pipe.Release(0)
        pipe.Release(0)                                        # nothing left to fence: no-op
        pipe.Release(5)                                        # not the slot's layer: no-op
