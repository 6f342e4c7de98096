"""Benchmark of the paged-KV attention path on one MI355X.

Default workload: Llama-3-8B-shape decode attention for one layer: 32 query
heads, 8 kv heads, head_dim 128, one query token over 32,768 cached tokens
(128 pages of 256), fp32 KV (the reference's page type), batch 1.  A step is
one attention call over one batch; the KV of consecutive steps rotates
through copies totalling more than 1 GB, so the 256 MB Infinity Cache cannot
serve repeats.  Inputs are synthetic N(0,1) (RoPE at base 500000 on Q and K)
generated on the device.

Prints one JSON line (rank 0, N=1).  `value` is the achieved HBM throughput
(algorithmic bytes per step / step time) in TB/s.  `roofline` is computed
for the dominant kernel from HIP events around the timed steps.
`cpu_baseline` times the oracle's op-order restatement of the reference's
single-threaded Vector256 path on one host core over a bounded sample.

Other workloads (--config): see WORKLOADS.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode attn µs/token & achieved HBM TB/s (% peak), 8B-shape @32K ctx, 1 GPU"
HBM_PEAK_TBS = 8.0
MFMA_PEAK_TFS = {"bf16": 2500.0, "f16": 2500.0}
ROTATE_BYTES = 1.1e9

WORKLOADS = {
    # name: kind, heads, kv_heads, head_dim, cached tokens, kv dtype, batch, [queries]
    "c1": dict(kind="decode", heads=8, kv=2, D=64, n=512, dtype="f32", B=1, rope=0.0,
               desc="tiny GQA decode, 8 q heads / 2 kv heads / head_dim 64, 512 cached fp32 tokens, batch 1"),
    "c2-f32-b1": dict(kind="decode", heads=32, kv=8, D=128, n=32768, dtype="f32", B=1, rope=500000.0,
                      desc="llama-3-8b-shape decode attention, 32 q heads / 8 kv heads / head_dim 128, "
                           "32768 cached tokens (128 pages), fp32 KV, batch 1"),
    "c2-f16-b1": dict(kind="decode", heads=32, kv=8, D=128, n=32768, dtype="f16", B=1, rope=500000.0,
                      desc="llama-3-8b-shape decode attention, 32768 cached tokens, fp16 KV, batch 1"),
    "c2-f32-b16": dict(kind="decode", heads=32, kv=8, D=128, n=32768, dtype="f32", B=16, rope=500000.0,
                       desc="llama-3-8b-shape decode attention, 32768 cached tokens, fp32 KV, batch 16"),
    "c2-f16-b16": dict(kind="decode", heads=32, kv=8, D=128, n=32768, dtype="f16", B=16, rope=500000.0,
                       desc="llama-3-8b-shape decode attention, 32768 cached tokens, fp16 KV, batch 16"),
    "c4-decode": dict(kind="decode", heads=64, kv=8, D=128, n=131072, dtype="f16", B=1, rope=0.0,
                      desc="llama-3-70b-shape decode attention, 64 q heads / 8 kv heads, 131072 cached fp16 tokens"),
    "c4-verify": dict(kind="chunk", heads=64, kv=8, D=128, n=131072, dtype="f16", B=1, rope=0.0, nq=8,
                      q_dtype="f16",
                      desc="llama-3-70b-shape speculative verify, 8 causal draft queries after 131072 fp16 tokens"),
    "c3-prefill": dict(kind="chunk", heads=32, kv=8, D=128, n=6144, dtype="bf16", B=1, rope=0.0, nq=2048,
                       q_dtype="bf16",
                       desc="llama-3-8b-shape chunked prefill, 2048 causal bf16 queries after 6144 cached tokens"),
    "f1-rope-append": dict(kind="rope", heads=32, kv=8, D=128, n=2048, pos0=6144, dtype="f16", B=1, rope=500000.0,
                           desc="fused RoPE + append of 2048 positions (8B shape: 32 q heads, 8 kv heads, "
                                "head_dim 128) into an fp16 cache at positions 6144..8191"),
    "c5-mla": dict(kind="mla", heads=128, kv_lora=512, rope_dim=64, n=16384, dtype="bf16", B=1,
                   desc="MLA absorbed decode, 128 heads, 512+64 latent, 16384 cached bf16 tokens"),
    "f2-mla-layer": dict(kind="mla_layer", heads=128, kv_lora=512, rope_dim=64, nope=128, vdim=128, n=16384,
                         dtype="bf16", kvb_fmt="BF16", B=1,
                         desc="MLA absorbed layer block for one token: q-absorb through bf16 W_UK, attention over "
                              "16384 cached bf16 latents (128 heads, 512+64), W_UV up-projection (nope 128, v 128)"),
    "f2-mla-layer-q8": dict(kind="mla_layer", heads=128, kv_lora=512, rope_dim=64, nope=128, vdim=128, n=16384,
                            dtype="bf16", kvb_fmt="Q8_0", B=1,
                            desc="MLA absorbed layer block as f2-mla-layer with the kvb weights in Q8_0"),
    "f3-matvec-q4k": dict(kind="matvec", wfmt="Q4_K", dtype="f32", B=1,
                          desc="fused dequant + dot MatVecs of one llama-3-8b layer for one token: wq, wk, wv, wo "
                               "(4096/1024 x 4096), gate, up (14336 x 4096), down (4096 x 14336), Q4_K weights; "
                               "wq/wk/wv and gate/up as grouped calls on their shared input"),
    "f3-matvec-q8": dict(kind="matvec", wfmt="Q8_0", dtype="f32", B=1,
                         desc="the f3-matvec-q4k projections with Q8_0 weights"),
    "f3-matvec-f16": dict(kind="matvec", wfmt="F16", dtype="f32", B=1,
                          desc="the f3-matvec-q4k projections with F16 weights"),
    "f4-stream-q4k": dict(kind="stream", wfmt="Q4_K", layers=8, budget=160 << 20, dtype="f32", B=1,
                          desc="weight streaming: 8 llama-3-8b-shape Q4_K layers (wq, wk, wv, wo, gate, up, down "
                               "and two norms) read from a .qw file in the page cache through the two HBM "
                               "prefetch slots, each layer's 7 MatVecs for one token (4 grouped calls) queued behind its upload"),
}
PCIE_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction

# llama-3-8b layer projections (rows, cols): wq, wk, wv, wo, gate, up, down
MATVEC_SHAPES = [(4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096), (14336, 4096), (14336, 4096),
                 (4096, 14336)]
W_FORMATS = {"F16": (1, 1, 2), "Q8_0": (4, 32, 34), "Q4_K": (6, 256, 144)}  # code, block, bytes


# projections that read one activation vector run as one grouped call (qr_matvec_group_dev):
# wq/wk/wv of the normed x and gate/up of the normed FFN input (StreamingEngine.cs:240-242,
# :605-606); wo and down alone
MATVEC_GROUPS = [[0, 1, 2], [3], [4, 5], [6]]


def matvec_bytes(w):
    code, bs, bb = W_FORMATS[w["wfmt"]]
    weights = sum(r * (c // bs) * bb + r * 4 for r, c in MATVEC_SHAPES)
    return weights + sum(MATVEC_SHAPES[g[0]][1] * 4 for g in MATVEC_GROUPS)  # x once per group


STREAM_NAMES = ["wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"]  # MATVEC_SHAPES order


def stream_layer_bytes(w):
    code, bs, bb = W_FORMATS[w["wfmt"]]
    return sum(r * (c // bs) * bb for r, c in MATVEC_SHAPES)


def write_stream_model(w, path):
    """The f4 .qw file: per layer attn_norm, wq, wk, wv, wo, ffn_norm, gate, up, down in the
    reference's plan order, random quant bytes under the fixed scales of synth_weights."""
    import numpy as np

    from qauntrunner_amd.store import ModelStoreBuilder

    code, bs, bb = W_FORMATS[w["wfmt"]]
    rng = np.random.default_rng(11)
    b = ModelStoreBuilder(path, {"arch": "llama", "dim": 4096, "layers": w["layers"], "ffn": 14336})
    plan = {}
    for l in range(w["layers"]):
        for k, (r, c) in enumerate(MATVEC_SHAPES):
            if k == 0:
                plan[f"l{l}.attn_norm"] = ((4096,), 0, 4096 * 4)
            if k == 4:
                plan[f"l{l}.ffn_norm"] = ((4096,), 0, 4096 * 4)
            plan[f"l{l}.{STREAM_NAMES[k]}"] = ((r, c), code, r * (c // bs) * bb)
    for name, (dims, fmt, size) in plan.items():
        b.Plan(name, dims, fmt, size)

    def body(name):
        dims, fmt, size = plan[name]
        if fmt == 0:
            return np.ones(dims[0], np.float32).view(np.uint8)
        raw = rng.integers(0, 256, (size // bb, bb), dtype=np.uint8)
        if w["wfmt"] == "Q8_0":
            raw[:, 0:2] = np.float16(0.05 / 127).reshape(1).view(np.uint8)
        else:
            raw[:, 0:2] = np.float16(0.05 / 15 / 32).reshape(1).view(np.uint8)
            raw[:, 2:4] = np.float16(0.05 / 63).reshape(1).view(np.uint8)
        return raw.reshape(-1)
    b.Commit(body)


KVB_FORMATS = {"F32": (0, 1, 4), "F16": (1, 1, 2), "BF16": (2, 1, 2), "Q8_0": (4, 32, 34)}  # code, block, bytes


def kvb_bytes(w):
    code, bs, bb = KVB_FORMATS[w["kvb_fmt"]]
    return w["heads"] * (w["nope"] + w["vdim"]) * (w["kv_lora"] // bs * bb)


def profiled_traffic(name):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 PMC summaries
    (a line `traffic_bytes_per_launch[<workload>]: <bytes>` under profiles/), else None."""
    import glob
    import re

    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.md"))):
        for line in open(path):
            m = re.match(r"traffic_bytes_per_launch\[([\w-]+)\]:\s*(\d+)", line.strip())
            if m and m.group(1) == name:
                return int(m.group(2))
    return None


def esize(dtype):
    return 4 if dtype == "f32" else 2


def algorithmic(w):
    """(bytes, flops) per step: K+V payload + Q + O + page table; 4*D flops per (query, key, head)."""
    if w["kind"] == "mla":
        width = w["kv_lora"] + w["rope_dim"]
        pages = math.ceil(w["n"] / 256)
        b = w["n"] * width * esize(w["dtype"]) + w["heads"] * width * 4 + w["heads"] * w["kv_lora"] * 4 + pages * 4
        f = 2 * w["heads"] * w["n"] * (width + w["kv_lora"])
        return b, f
    if w["kind"] == "matvec":
        # every weight byte once + x in + y out per matrix; 2 flops per weight
        return matvec_bytes(w), sum(2 * r * c for r, c in MATVEC_SHAPES)
    if w["kind"] == "stream":
        # the weight bytes staged from the file per forward (norms stay unstaged), 2 flops per weight
        return w["layers"] * stream_layer_bytes(w), w["layers"] * sum(2 * r * c for r, c in MATVEC_SHAPES)
    if w["kind"] == "mla_layer":
        # latents + every kvb row once + q in + out; the q~/u hand-offs between kernels are not counted
        width = w["kv_lora"] + w["rope_dim"]
        pages = math.ceil(w["n"] / 256)
        H, nope, vdim, L = w["heads"], w["nope"], w["vdim"], w["kv_lora"]
        b = (w["n"] * width * esize(w["dtype"]) + kvb_bytes(w) + H * (nope + w["rope_dim"]) * 4 + H * vdim * 4
             + pages * 4)
        f = 2 * H * w["n"] * (width + L) + 2 * H * (nope + vdim) * L
        return b, f
    if w["kind"] == "rope":
        # read q, k, v (fp32), write q (fp32) and k, v (cache dtype); 6 flops per rotated pair
        n, kvd, qd = w["n"], w["kv"] * w["D"], w["heads"] * w["D"]
        b = n * (2 * qd * 4 + 2 * kvd * 4 + 2 * kvd * esize(w["dtype"])) + math.ceil(n / 256) * 4
        f = n * (qd + kvd) // 2 * 6
        return b, f
    nq = w.get("nq", 1)
    total = w["n"] + (nq if w["kind"] == "chunk" else 0)
    pages = math.ceil(total / 256)
    kv_bytes = 2 * total * w["kv"] * w["D"] * esize(w["dtype"])
    qe = esize(w.get("q_dtype", "f32"))
    b = w["B"] * (kv_bytes + nq * w["heads"] * w["D"] * (qe + 4) + pages * 4)
    keys = sum(w["n"] + i + 1 for i in range(nq)) if w["kind"] == "chunk" else w["n"]
    f = w["B"] * 4 * w["D"] * w["heads"] * keys
    return b, f


def rope_(x, D, pos0, theta):
    """Rotate-half RoPE in fp32 on rows [n, heads*D], row r at position pos0+r (input synthesis only)."""
    import torch

    if theta == 0.0:
        return x
    n = x.shape[0]
    half = D // 2
    inv = torch.pow(torch.tensor(theta, dtype=torch.float64), -2.0 * torch.arange(half, dtype=torch.float64) / D)
    ang = (torch.arange(n, dtype=torch.float64) + pos0)[:, None] * inv[None, :]
    c = torch.cos(ang).float().to(x.device)[:, None, :]
    s = torch.sin(ang).float().to(x.device)[:, None, :]
    v = x.view(n, -1, D)
    a, b = v[..., :half].clone(), v[..., half:].clone()
    v[..., :half] = a * c - b * s
    v[..., half:] = a * s + b * c
    return x


def to_cache_bits(x, dtype):
    import torch

    if dtype == "f32":
        return x.contiguous()
    t = x.half() if dtype == "f16" else x.bfloat16()
    return t.contiguous().view(torch.int16)


def prepared(fn, *args):
    """One C-ABI call with its ctypes arguments converted once, so that the timed loop
    pays the library's own host work and the launches, not Python argument handling
    (a decode call is ~50 us of GPU time; building the arguments per call took longer)."""
    import ctypes

    from qauntrunner_amd._lib import check

    conv = [a if isinstance(a, (ctypes._SimpleCData, ctypes.Array)) else
            ctypes.c_void_p(a) if isinstance(a, int) and a > 1 << 20 else a for a in args]

    def call():
        st = fn(*conv)
        if st:
            check(st)
    return call


def np_i32(values):
    import numpy as np

    return np.ascontiguousarray(values, dtype=np.int32)


def build_decode(w, gen, dev):
    """KV handle with R rotation sets of B sequences each, filled on the device."""
    import torch

    import qauntrunner_amd as qr

    nq = w.get("nq", 1)
    total = w["n"] + (nq if w["kind"] == "chunk" else 0)
    set_bytes = w["B"] * 2 * total * w["kv"] * w["D"] * esize(w["dtype"])
    R = max(1, math.ceil(ROTATE_BYTES / set_bytes))
    kv = qr.PagedKvCache(1, w["heads"], w["kv"], w["D"], total, kv_dtype=w["dtype"], max_batch=R * w["B"])
    kv.Reserve(R * w["B"] * math.ceil(total / 256))
    kv_dim = w["kv"] * w["D"]
    chunk = 8192
    for s in range(R * w["B"]):
        for p0 in range(0, total, chunk):
            m = min(chunk, total - p0)
            K = rope_(torch.randn(m, kv_dim, device=dev, generator=gen), w["D"], p0, w["rope"])
            V = torch.randn(m, kv_dim, device=dev, generator=gen)
            kv.AppendRangeDev(0, p0, to_cache_bits(K, w["dtype"]), to_cache_bits(V, w["dtype"]),
                              src_dtype=w["dtype"], seq_id=s)
    torch.cuda.synchronize()
    return kv, R


def run_gpu(w, steps, warmup):
    import ctypes

    import torch

    import qauntrunner_amd as qr

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1234)
    stream = torch.cuda.current_stream()

    if w["kind"] == "mla":
        width = w["kv_lora"] + w["rope_dim"]
        set_bytes = w["n"] * width * esize(w["dtype"])
        R = max(1, math.ceil(ROTATE_BYTES / set_bytes))
        cache = qr.MlaLatentCache(R, w["kv_lora"] + w["rope_dim"], w["n"], dtype=w["dtype"], rope=w["rope_dim"])
        cache.Reserve(R * math.ceil(w["n"] / 256))
        for layer in range(R):
            rows = torch.randn(w["n"], width, device=dev, generator=gen)
            cache.AppendRangeDev(layer, 0, to_cache_bits(rows, w["dtype"]), src_dtype=w["dtype"])
        qt = torch.randn(R, w["heads"], w["kv_lora"], device=dev, generator=gen)
        qrp = torch.randn(R, w["heads"], w["rope_dim"], device=dev, generator=gen)
        u = torch.empty(R, w["heads"], w["kv_lora"], device=dev)
        scale = 1.0 / math.sqrt(192.0)

        cache.AbsorbedAttentionDev(0, w["n"] - 1, qt[0], qrp[0], u[0], scale, stream=stream)  # checks shapes once
        sp = stream.cuda_stream
        calls = [prepared(cache._lib.qr_mla_attention_dev, cache._h, r, w["n"] - 1, w["heads"], qt[r].data_ptr(),
                          qrp[r].data_ptr(), ctypes.c_float(scale), u[r].data_ptr(), ctypes.c_void_p(sp))
                 for r in range(R)]

        def step(i):
            calls[i % R]()
        handle = cache
    elif w["kind"] == "mla_layer":
        width = w["kv_lora"] + w["rope_dim"]
        H, nope, vdim, L = w["heads"], w["nope"], w["vdim"], w["kv_lora"]
        code = KVB_FORMATS[w["kvb_fmt"]][0]
        set_bytes = w["n"] * width * esize(w["dtype"]) + kvb_bytes(w)
        R = max(1, math.ceil(ROTATE_BYTES / set_bytes))
        cache = qr.MlaLatentCache(R, L + w["rope_dim"], w["n"], dtype=w["dtype"], rope=w["rope_dim"])
        cache.Reserve(R * math.ceil(w["n"] / 256))
        kvbs = []
        for layer in range(R):
            rows = torch.randn(w["n"], width, device=dev, generator=gen)
            cache.AppendRangeDev(layer, 0, to_cache_bits(rows, w["dtype"]), src_dtype=w["dtype"])
            kvbs.append(synth_kvb(w, gen, dev))
        q = torch.randn(R, H, nope + w["rope_dim"], device=dev, generator=gen)
        out = torch.empty(R, H, vdim, device=dev)

        cache.AttendAbsorbedDev(0, w["n"] - 1, q[0], kvbs[0], code, nope, vdim, out[0], stream=stream)
        sp = stream.cuda_stream
        calls = [prepared(cache._lib.qr_mla_attend_absorbed_dev, cache._h, r, w["n"] - 1, H, nope, vdim,
                          q[r].data_ptr(), kvbs[r].data_ptr(), code, out[r].data_ptr(), ctypes.c_void_p(sp))
                 for r in range(R)]

        def step(i):
            calls[i % R]()
        handle = cache
        proj = {"absorb": lambda r: qr.mla_q_absorb_dev(kvbs[r], code, H, nope, w["rope_dim"], vdim, L, q[r],
                                                        qt_scratch[r], stream=stream),
                "wuv": lambda r: qr.mla_wuv_dev(kvbs[r], code, H, nope, vdim, L, qt_scratch[r], out[r],
                                                stream=stream)}
        qt_scratch = torch.randn(R, H, L, device=dev, generator=gen)
    elif w["kind"] == "matvec":
        code, bs, bb = W_FORMATS[w["wfmt"]]
        set_bytes = matvec_bytes(w)
        R = max(1, math.ceil(ROTATE_BYTES / set_bytes))
        mats = [[synth_weights(w["wfmt"], r, c, gen, dev) for r, c in MATVEC_SHAPES] for _ in range(R)]
        xs = [torch.randn(c, device=dev, generator=gen) for _, c in MATVEC_SHAPES]
        ys = [torch.empty(r, device=dev) for r, _ in MATVEC_SHAPES]

        for g in MATVEC_GROUPS:
            qr.matvec_group_dev([mats[0][k] for k in g], code, [MATVEC_SHAPES[k][0] for k in g],
                                MATVEC_SHAPES[g[0]][1], xs[g[0]], [ys[k] for k in g], stream=stream)
        lib = qr.load()
        sp = ctypes.c_void_p(stream.cuda_stream)

        def group_call(m, g):
            n = len(g)
            wp = (ctypes.c_void_p * n)(*[m[k].data_ptr() for k in g])
            rp = (ctypes.c_longlong * n)(*[MATVEC_SHAPES[k][0] for k in g])
            yp = (ctypes.c_void_p * n)(*[ys[k].data_ptr() for k in g])
            return prepared(lib.qr_matvec_group_dev, n, wp, rp, code, MATVEC_SHAPES[g[0]][1], 1, xs[g[0]].data_ptr(),
                            yp, sp)
        calls = [[group_call(m, g) for g in MATVEC_GROUPS] for m in mats]

        def step(i):
            for call in calls[i % R]:
                call()

        class _NoHandle:
            def close(self):
                pass
        handle = _NoHandle()
    elif w["kind"] == "stream":
        import tempfile

        code = W_FORMATS[w["wfmt"]][0]
        tmpdir = tempfile.mkdtemp(prefix="qr_stream_")
        path = os.path.join(tmpdir, "layers.qw")
        write_stream_model(w, path)
        xs = [torch.randn(c, device=dev, generator=gen) for _, c in MATVEC_SHAPES]
        ys = [torch.empty(r, device=dev) for r, _ in MATVEC_SHAPES]
        L = w["layers"]

        def forward(p):
            """StreamingEngine.Forward's weight order (StreamingEngine.cs:225-266)."""
            p.Begin(0)
            for l in range(L):
                wts = [p.Acquire(f"l{l}.{STREAM_NAMES[k]}", l, stream) for k in range(len(MATVEC_SHAPES))]
                for g in MATVEC_GROUPS:
                    qr.matvec_group_dev([wts[k] for k in g], code, [MATVEC_SHAPES[k][0] for k in g],
                                        MATVEC_SHAPES[g[0]][1], xs[g[0]], [ys[k] for k in g], stream=stream)
                p.Release(l, stream)
                if l + 1 < L:
                    p.Begin(l + 1)

        store = qr.ModelStore.Open(path)
        pipe = qr.PrefetchPipeline(store, w["budget"])

        def step(i):
            forward(pipe)

        class _Stream:
            def close(self):
                store.Dispose()
                os.remove(path)
                os.rmdir(tmpdir)
        handle = _Stream()

        def resident_and_upload(steps, warmup):
            """The same forward with every tensor resident (the MatVecs alone), and the pinned
            host-to-device copy rate of one layer's bytes."""
            out = {}
            with qr.ModelStore.Open(path) as rs:
                rp = qr.PrefetchPipeline(rs, w["budget"])
                rs.MakeResident()
                for _ in range(warmup):
                    forward(rp)
                torch.cuda.synchronize()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                for _ in range(steps):
                    forward(rp)
                b.record(stream)
                torch.cuda.synchronize()
                out["resident_ms"] = a.elapsed_time(b) / steps
            host = torch.empty(stream_layer_bytes(w), dtype=torch.uint8, pin_memory=True)
            devb = torch.empty_like(host, device=dev)
            for _ in range(3):
                devb.copy_(host, non_blocking=True)
            torch.cuda.synchronize()
            a.record(stream)
            for _ in range(10):
                devb.copy_(host, non_blocking=True)
            b.record(stream)
            torch.cuda.synchronize()
            out["h2d_GBs"] = host.numel() * 10 / (a.elapsed_time(b) * 1e-3) / 1e9
            out["host_read_GBs"] = host_read_rate(path, host.numpy())
            return out
    elif w["kind"] == "rope":
        n, kvd, qd = w["n"], w["kv"] * w["D"], w["heads"] * w["D"]
        set_bytes = n * (qd + 2 * kvd) * 4
        R = max(1, math.ceil(ROTATE_BYTES / set_bytes))
        kv = qr.PagedKvCache(1, w["heads"], w["kv"], w["D"], w["pos0"] + n, kv_dtype=w["dtype"], max_batch=R)
        kv.Reserve(R * math.ceil((w["pos0"] + n) / 256))
        qs = torch.randn(R, n, qd, device=dev, generator=gen)
        ks = torch.randn(R, n, kvd, device=dev, generator=gen)
        vs = torch.randn(R, n, kvd, device=dev, generator=gen)

        for r in range(R):  # pages assigned and shapes checked once; the timed calls rewrite them
            kv.AppendRopeDev(0, w["pos0"], qs[r], ks[r], vs[r], w["rope"], seq_id=r, stream=stream)
        sp = stream.cuda_stream
        calls = [prepared(kv._lib.qr_kv_append_rope_dev, kv._h, r, 0, w["pos0"], n, qs[r].data_ptr(),
                          ks[r].data_ptr(), vs[r].data_ptr(), ctypes.c_float(w["rope"]), ctypes.c_void_p(sp))
                 for r in range(R)]

        def step(i):
            calls[i % R]()
        handle = kv
    else:
        kv, R = build_decode(w, gen, dev)
        B = w["B"]
        nq = w.get("nq", 1)
        row = w["heads"] * w["D"]
        scale = 1.0 / math.sqrt(w["D"])
        if w["kind"] == "decode":
            q = rope_(torch.randn(R * B, row, device=dev, generator=gen), w["D"], w["n"] - 1, w["rope"])
            out = torch.empty(R * B, row, device=dev)

            kv.AttentionDev(0, list(range(B)), [w["n"] - 1] * B, q[:B], out[:B], scale, stream=stream)
            ids = [np_i32(range(r * B, (r + 1) * B)) for r in range(R)]
            pos = np_i32([w["n"] - 1] * B)
            calls = [prepared(kv._lib.qr_kv_attention_dev, kv._h, B, ids[r].ctypes.data, 0, pos.ctypes.data,
                              q[r * B].data_ptr(), out[r * B].data_ptr(), ctypes.c_float(scale),
                              ctypes.c_void_p(stream.cuda_stream)) for r in range(R)]
        else:
            q = to_cache_bits(torch.randn(R, nq, row, device=dev, generator=gen), w["q_dtype"])
            out = torch.empty(R, nq, row, device=dev)
            kv.AttentionChunkDev(0, w["n"], q[0], out[0], scale, q_dtype=w["q_dtype"], seq_id=0, stream=stream)
            calls = [prepared(kv._lib.qr_kv_attention_chunk_dev, kv._h, r, 0, w["n"], nq, q[r].data_ptr(),
                              qr.dtype_code(w["q_dtype"]), out[r].data_ptr(), ctypes.c_float(scale),
                              ctypes.c_void_p(stream.cuda_stream)) for r in range(R)]

        def step(i):
            calls[i % R]()
        handle = kv

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    wall0 = time.perf_counter()
    for i in range(steps):
        step(warmup + i)
    wall = time.perf_counter() - wall0  # host time to enqueue the steps (the GPU runs behind)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    kernel_ms = None
    if hasattr(handle, "SetSplitEvent") and w["kind"] != "rope":
        kernel_ms = time_split_kernel(handle, step, warmup + steps, steps, stream)
    extra = None
    if w["kind"] == "mla_layer":
        extra = {}
        for name, fn in proj.items():
            for i in range(warmup):
                fn(i % R)
            t0.record(stream)
            for i in range(steps):
                fn((warmup + i) % R)
            t1.record(stream)
            torch.cuda.synchronize()
            extra[name] = t0.elapsed_time(t1) / steps
    if w["kind"] == "stream":
        extra = resident_and_upload(max(1, steps // 2), max(1, warmup // 2))
        extra.update(zip(("bytes_streamed", "wait_ms", "read_ms", "staged", "skipped"),
                         (pipe.BytesStreamed, pipe.WaitMs, pipe.ReadMs, pipe.StagedLayers, pipe.SkippedLayers)))
    handle.close()
    return ms, wall * 1e3 / steps, kernel_ms, extra


def host_read_rate(path, pinned, threads=16, chunk=2 << 20, repeats=5):
    """GB/s of positional reads of the file's first len(pinned) bytes into a pinned host buffer
    by `threads` threads in `chunk` pieces (the staging reads alone; median of `repeats`)."""
    import threading

    n = pinned.size
    view = memoryview(pinned)
    fd = os.open(path, os.O_RDONLY)
    rates = []
    try:
        for _ in range(repeats):
            nxt = [0]
            lock = threading.Lock()

            def work():
                while True:
                    with lock:
                        i = nxt[0]
                        nxt[0] += chunk
                    if i >= n:
                        return
                    os.preadv(fd, [view[i:min(n, i + chunk)]], i)
            pool = [threading.Thread(target=work) for _ in range(threads)]
            t = time.perf_counter()
            for th in pool:
                th.start()
            for th in pool:
                th.join()
            rates.append(n / (time.perf_counter() - t) / 1e9)
    finally:
        os.close(fd)
    return sorted(rates)[len(rates) // 2]


def synth_weights(fmt, rows, cols, gen, dev):
    """rows x cols weights in fmt as a uint8 device tensor: N(0, 0.05^2) for F16; for the block
    formats random quant bytes under small fixed f16 scales (every byte pattern is a valid
    block once the scale fields are finite)."""
    import torch

    if fmt == "F16":
        return (torch.randn(rows, cols, device=dev, generator=gen) * 0.05).half().view(torch.uint8).reshape(-1)
    code, bs, bb = W_FORMATS[fmt]
    blocks = rows * cols // bs
    raw = torch.randint(0, 256, (blocks, bb), dtype=torch.uint8, device=dev, generator=gen)
    if fmt == "Q8_0":
        raw[:, 0:2] = torch.full((blocks,), 0.05 / 127, dtype=torch.float16, device=dev).view(torch.uint8).view(blocks, 2)
    else:  # Q4_K: d, dmin
        raw[:, 0:2] = torch.full((blocks,), 0.05 / 15 / 32, dtype=torch.float16, device=dev).view(torch.uint8).view(blocks, 2)
        raw[:, 2:4] = torch.full((blocks,), 0.05 / 63, dtype=torch.float16, device=dev).view(torch.uint8).view(blocks, 2)
    return raw.reshape(-1)


def synth_kvb(w, gen, dev):
    """kvb rows [heads*(nope+vdim)][kv_lora] in the workload's format, N(0, 0.05^2) weights
    (Q8_0: random int8 values under an f16 scale of 0.05/127), as a uint8 device tensor."""
    import torch

    rows = w["heads"] * (w["nope"] + w["vdim"])
    L = w["kv_lora"]
    fmt = w["kvb_fmt"]
    if fmt == "Q8_0":
        blocks = rows * L // 32
        raw = torch.randint(0, 256, (blocks, 34), dtype=torch.uint8, device=dev, generator=gen)
        d = torch.full((blocks,), 0.05 / 127, dtype=torch.float16, device=dev)
        raw[:, 0:2] = d.view(torch.uint8).view(blocks, 2)
        return raw.reshape(-1)
    x = torch.randn(rows, L, device=dev, generator=gen) * 0.05
    if fmt == "F32":
        return x.view(torch.uint8).reshape(-1)
    return to_cache_bits(x, "f16" if fmt == "F16" else "bf16").view(torch.uint8).reshape(-1)


def stream_floor_us(nbytes, steps, warmup):
    """Average time of a plain streaming read of `nbytes` (libqr_floor.so: every byte read
    once with non-temporal 16-byte loads, nothing computed), launched back to back over
    rotated buffers of at least ROTATE_BYTES in all, as the workloads rotate their data; the
    faster of 256 and 512 workgroups.  What HBM gives a kernel that does nothing but read,
    on this GPU in this process.  None when the helper library is not built."""
    import ctypes

    import torch

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qauntrunner_amd", "libqr_floor.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.qr_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_int, ctypes.c_void_p]
    n = (int(nbytes) + 4095) // 4096 * 4096
    sets = max(1, math.ceil(ROTATE_BYTES / n))
    buf = torch.ones(sets * n, dtype=torch.uint8, device="cuda:0")
    sink = torch.zeros(64, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    best = None
    for blocks in (256, 512):
        def launch(reps):
            rc = lib.qr_floor_read(buf.data_ptr(), n, sets, reps, sink.data_ptr(), blocks, stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"qr_floor_read returned {rc}")
        launch(max(1, warmup))
        torch.cuda.synchronize()
        t0.record(stream)
        launch(steps)
        t1.record(stream)
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / steps * nbytes / n
        best = us if best is None else min(best, us)
    del buf
    return best


def time_split_kernel(handle, step, first, steps, stream):
    """Average duration of the split-K kernel alone: per step, a HIP event is recorded
    on the launch stream before the call and the library records another right after
    the split-K kernel (before the combine)."""
    import ctypes

    import torch

    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
    hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
    sptr = ctypes.c_void_p(stream.cuda_stream)
    starts, mids = [], []
    for _ in range(steps):
        for lst in (starts, mids):
            e = ctypes.c_void_p()
            assert hip.hipEventCreate(ctypes.byref(e)) == 0
            lst.append(e)
    torch.cuda.synchronize()
    for i in range(steps):
        assert hip.hipEventRecord(starts[i], sptr) == 0
        handle.SetSplitEvent(mids[i])
        step(first + i)
    handle.SetSplitEvent(None)
    torch.cuda.synchronize()
    total = 0.0
    for a, b in zip(starts, mids):
        f = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(f), a, b) == 0
        total += f.value
    for e in starts + mids:
        hip.hipEventDestroy(e)
    return total / steps


def host_info():
    """nproc, CPU model and clock of this host (from /proc/cpuinfo)."""
    model, mhz = "unknown", []
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("cpu MHz"):
                    mhz.append(float(line.split(":", 1)[1]))
    except OSError:
        pass
    clock = f"{max(mhz):.0f} MHz (max of the cores' current clocks)" if mhz else "clock unknown"
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity")
            else None, "cpu_model": model, "clock": clock}


def cpu_baseline(w, budget_s=10.0):
    """Oracle (op-order restatement of the reference's single-threaded path) on one core."""
    import numpy as np

    from oracle import oracle

    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except (AttributeError, OSError):
        pass
    hi = host_info()
    rng = np.random.default_rng(7)
    bytes_step, _ = algorithmic(w)
    if w["kind"] == "rope":
        sample_rows = 64
        qd, kvd = w["heads"] * w["D"], w["kv"] * w["D"]
        Q = rng.standard_normal((sample_rows, qd), dtype=np.float32)
        K = rng.standard_normal((sample_rows, kvd), dtype=np.float32)
        V = rng.standard_normal((sample_rows, kvd), dtype=np.float32)
        pages = np.zeros((2, sample_rows, kvd), np.float32)

        def call():  # BuildCosSin + Rope on q and k, then the row copies of Append
            qr_ = oracle.rope_rows(Q, w["D"], w["pos0"], w["rope"])
            kr = oracle.rope_rows(K, w["D"], w["pos0"], w["rope"])
            pages[0] = kr
            pages[1] = V
            return qr_
        unit_fraction = sample_rows / w["n"]
        sample = f"{sample_rows} of {w['n']} positions, fp32 storage"
    elif w["kind"] == "stream":
        return cpu_stream_baseline(w, budget_s)
    elif w["kind"] == "matvec":
        code, bs, bb = W_FORMATS[w["wfmt"]]
        sample_rows = 32
        mats = []
        for r, c in MATVEC_SHAPES:
            if w["wfmt"] == "F16":
                raw = (rng.standard_normal((sample_rows, c)) * 0.05).astype(np.float16).view(np.uint8)
            else:  # random quant bytes under the same fixed scales as the device synthesis
                raw = rng.integers(0, 256, (sample_rows * c // bs, bb), dtype=np.uint8)
                if w["wfmt"] == "Q8_0":
                    raw[:, 0:2] = np.float16(0.05 / 127).reshape(1).view(np.uint8)
                else:
                    raw[:, 0:2] = np.float16(0.05 / 15 / 32).reshape(1).view(np.uint8)
                    raw[:, 2:4] = np.float16(0.05 / 63).reshape(1).view(np.uint8)
            mats.append((np.ascontiguousarray(raw).reshape(sample_rows, -1), c,
                         rng.standard_normal(c).astype(np.float32)))
        total_rows = sum(r for r, _ in MATVEC_SHAPES)

        def call():  # DotRow over a sample of every matrix's rows
            for raw, c, x in mats:
                oracle.matvec(code, raw, c, x)
        unit_fraction = len(MATVEC_SHAPES) * sample_rows / total_rows
        sample = (f"DotRow over {sample_rows} rows of each of the 7 matrices ({len(MATVEC_SHAPES) * sample_rows} of "
                  f"{total_rows} rows), scaled to all rows")
    elif w["kind"] == "mla_layer":
        width = w["kv_lora"] + w["rope_dim"]
        H, nope, vdim, L, rp = w["heads"], w["nope"], w["vdim"], w["kv_lora"], w["rope_dim"]
        heads_sample = 4
        lat = rng.standard_normal((w["n"], width), dtype=np.float32)
        kvb = (rng.standard_normal((heads_sample * (nope + vdim), L), dtype=np.float32) * 0.05)
        q = rng.standard_normal((heads_sample, nope + rp), dtype=np.float32)
        scale = 1 / math.sqrt(nope + rp)

        def call():  # absorb, attention, W_UV for a sample of heads (kvb already decoded)
            qt = oracle.mla_q_absorb(q, kvb, heads_sample, nope, rp, vdim, L)
            u = oracle.mla_attention(lat, qt, q[:, nope:], L, rp, scale)
            return oracle.mla_wuv(u, kvb, heads_sample, nope, vdim, L)
        unit_fraction = heads_sample / H
        sample = (f"absorb + attention over {w['n']} tokens + W_UV for {heads_sample} of {H} heads, "
                  "scaled to all heads, kvb pre-decoded to fp32")
    elif w["kind"] == "mla":
        width = w["kv_lora"] + w["rope_dim"]
        lat = rng.standard_normal((w["n"], width), dtype=np.float32)
        qt = rng.standard_normal((w["heads"], w["kv_lora"]), dtype=np.float32)
        qrp = rng.standard_normal((w["heads"], w["rope_dim"]), dtype=np.float32)
        heads_sample = 8
        def call():
            oracle.mla_attention(lat, qt[:heads_sample], qrp[:heads_sample], w["kv_lora"], w["rope_dim"], 0.072)
        unit_fraction = heads_sample / w["heads"]
        sample = f"MLA over {w['n']} tokens for {heads_sample} of {w['heads']} heads, scaled to all heads"
    else:
        nq = w.get("nq", 1)
        total = w["n"] + (nq if w["kind"] == "chunk" else 0)
        K = rng.standard_normal((total, w["kv"] * w["D"]), dtype=np.float32)
        V = rng.standard_normal((total, w["kv"] * w["D"]), dtype=np.float32)
        q = rng.standard_normal(w["heads"] * w["D"], dtype=np.float32)
        seq = w["n"] + (nq // 2 if w["kind"] == "chunk" else 0)
        def call():
            oracle.kv_attention(K[:seq], V[:seq], q, w["heads"], w["kv"], w["D"], 1 / math.sqrt(w["D"]))
        unit_fraction = 1.0 / (w["B"] * nq)
        sample = (f"one query over {seq} tokens (a 1/{w['B'] * nq} share of the step), "
                  "fp32 storage of the same values")
    times = []
    start = time.perf_counter()
    while True:
        t = time.perf_counter()
        call()
        times.append(time.perf_counter() - t)
        if time.perf_counter() - start > budget_s or len(times) >= 200:
            break
    times.sort()
    med = times[len(times) // 2]
    step_s = med / unit_fraction
    tokens = w.get("B", 1) * w.get("nq", 1)
    return {
        "value": bytes_step / step_s / 1e12,
        "unit": "TB/s",
        "cores": 1,
        "kind": "port",
        "ms_per_step": round(step_s * 1e3, 3),
        "us_per_token": round(step_s * 1e6 / tokens, 1),
        "sample": f"{sample}; median of {len(times)} calls ({med * 1e3:.1f} ms each), "
                  f"step {step_s * 1e3:.1f} ms; one core pinned of nproc {hi['nproc']} "
                  f"({hi['affinity']} in this process's affinity), {hi['cpu_model']}, {hi['clock']}",
        "host": hi,
    }


def cpu_stream_baseline(w, budget_s):
    """The reference's CPU forward over streamed weights, per layer: ReadLayer's positional reads
    of the layer into one host buffer (PrefetchPipeline.cs:146-153, one thread, page cache) plus
    DotRow over every row (sampled as in the matvec leg); the layer time times the layer count."""
    import tempfile

    import numpy as np

    layer = stream_layer_bytes(w)
    tmpdir = tempfile.mkdtemp(prefix="qr_cpu_stream_")
    path = os.path.join(tmpdir, "layer.bin")
    rng = np.random.default_rng(5)
    with open(path, "wb") as f:
        f.write(rng.integers(0, 256, layer, dtype=np.uint8).tobytes())
    buf = bytearray(layer)
    view = memoryview(buf)
    fd = os.open(path, os.O_RDONLY)
    reads = []
    try:
        start = time.perf_counter()
        while time.perf_counter() - start < budget_s / 2 and len(reads) < 20:
            t = time.perf_counter()
            done = 0
            while done < layer:
                done += os.preadv(fd, [view[done:done + (64 << 20)]], done)
            reads.append(time.perf_counter() - t)
    finally:
        os.close(fd)
        os.remove(path)
        os.rmdir(tmpdir)
    reads.sort()
    read_s = reads[len(reads) // 2]
    mv = cpu_baseline(dict(w, kind="matvec"), budget_s / 2)
    matvec_s = matvec_bytes(w) / (mv["value"] * 1e12)
    step_s = w["layers"] * (read_s + matvec_s)
    bytes_step, _ = algorithmic(w)
    return {
        "value": bytes_step / step_s / 1e12,
        "unit": "TB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"per layer: {layer / 1e6:.1f} MB read from the page cache in {read_s * 1e3:.1f} ms "
                   f"(median of {len(reads)}) + DotRow over all rows {matvec_s * 1e3:.1f} ms "
                   f"({mv['sample']}); step = {w['layers']} layers, {step_s * 1e3:.1f} ms"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2-f32-b1", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 1 GiB device-to-device copy (scales rocprofv3 FETCH_SIZE/WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch

        x = torch.empty(1 << 28, dtype=torch.float32, device="cuda:0").fill_(1.0)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": x.numel() * 4, "bytes_written": y.numel() * 4}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only; --gpus {args.gpus} is not supported "
              "(the kernels are the one-GPU share at its real shape; no multi-GPU path exists)", file=sys.stderr)
        sys.exit(2)

    w = WORKLOADS[args.config]
    ms, wall_ms, kernel_ms, extra = run_gpu(w, args.steps, args.warmup)
    bytes_step, flops_step = algorithmic(w)
    tbs = bytes_step / (ms * 1e-3) / 1e12
    # The attention call (split-K kernel + split merge, as the metric defines it): the
    # timed loop is device-bound (host time per step is reported beside it), so the HIP
    # events around the timed steps measure the kernels back to back.
    kms = ms
    nq = w.get("nq", 1)
    tokens = w["B"] * nq
    dtype = w["dtype"]
    mfma = w["kind"] == "chunk" and nq > 64
    if mfma:
        achieved = flops_step / (kms * 1e-3) / 1e12
        roof = {"bound": "mfma", "achieved": achieved, "peak": MFMA_PEAK_TFS.get(dtype, 2500.0),
                "unit": "TFLOP/s", "frac": achieved / MFMA_PEAK_TFS.get(dtype, 2500.0), "traffic": None}
    else:
        achieved = bytes_step / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_TBS * 1e3, "unit": "GB/s",
                "frac": achieved / (HBM_PEAK_TBS * 1e3), "traffic": None}
    if w["kind"] == "stream":
        # the kernels of the step are the MatVecs; timed with every tensor resident
        kms = extra["resident_ms"]
        mv_bytes = w["layers"] * matvec_bytes(w)
        achieved = mv_bytes / (kms * 1e-3) / 1e9
        roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_TBS * 1e3, "unit": "GB/s",
                "frac": achieved / (HBM_PEAK_TBS * 1e3), "traffic": None}
    roof["traffic"] = profiled_traffic(args.config)
    roof["kernel_us"] = round(kms * 1e3, 3)
    if roof["bound"] == "hbm" and w["kind"] != "rope":
        # the same bytes read by a kernel that does nothing else (rope writes half its bytes)
        floor = stream_floor_us(roof["achieved"] * 1e9 * kms * 1e-3, args.steps, args.warmup)
        if floor is not None:
            roof["stream_floor_us"] = round(floor, 3)
            roof["floor_frac"] = round(floor / (kms * 1e3), 4)
    roof["kernel"] = ("attention call: split-K kernel + split merge (inside the split-K kernel for decode "
                      "plans whose splits fit one pass of the GPU, else a merge kernel; HIP events around the "
                      "timed steps on the launch stream)" if w["kind"] in ("decode", "chunk", "mla") else
                      "whole step (HIP events around the timed steps on the launch stream)")
    if kernel_ms:
        roof["split_kernel_us"] = round(kernel_ms * 1e3, 3)
    if w["kind"] == "stream":
        roof["kernel"] = (f"the {7 * w['layers']} MatVecs ({len(MATVEC_GROUPS) * w['layers']} grouped launches) of a "
                          "resident forward (HIP events)")
    line = {
        "metric": METRIC,
        "value": round(tbs, 4),
        "unit": "TB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "us_per_token": round(ms * 1e3 / tokens, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": ("synthetic Q4_K blocks (random quants, fixed scales) in a .qw file in the page cache"
                 if w["kind"] == "stream" else
                 "synthetic N(0,1) on device" + (", RoPE base 500000 on Q/K" if w.get("rope") else "")),
        "config": {"workload": w["desc"], "name": args.config, "algorithmic_bytes": bytes_step,
                   "algorithmic_flops": flops_step, "host_enqueue_ms_per_step": round(wall_ms, 4)},
        "roofline": roof,
    }
    if w["kind"] == "stream":
        streamed = bytes_step / (ms * 1e-3) / 1e9
        line["stream"] = {
            "staged_GBs": round(streamed, 2), "peak_GBs": PCIE_PEAK_GBS, "peak": "PCIe 5.0 x16, one direction",
            "frac": round(streamed / PCIE_PEAK_GBS, 4),
            "h2d_pinned_GBs": round(extra["h2d_GBs"], 2),
            "host_read_pinned_GBs": round(extra["host_read_GBs"], 2),
            "resident_ms_per_step": round(extra["resident_ms"], 4),
            "layer_bytes": stream_layer_bytes(w), "budget": w["budget"],
            "host_wait_ms_total": round(extra["wait_ms"], 2), "host_read_ms_total": round(extra["read_ms"], 2),
            "bytes_streamed_total": extra["bytes_streamed"], "staged_layers": extra["staged"],
            "skipped_layers": extra["skipped"]}
    elif extra:
        # the projection kernels timed alone (HIP events around `steps` launches each)
        H, nope, vdim, L = w["heads"], w["nope"], w["vdim"], w["kv_lora"]
        per_row = kvb_bytes(w) // (H * (nope + vdim))
        proj_bytes = {"absorb": H * nope * per_row + H * (nope + w["rope_dim"]) * 4 + H * L * 4,
                      "wuv": H * vdim * per_row + H * L * 4 + H * vdim * 4}
        line["projections"] = {
            k: {"kernel_us": round(v * 1e3, 3), "algorithmic_bytes": proj_bytes[k],
                "achieved_GBs": round(proj_bytes[k] / (v * 1e-3) / 1e9, 1),
                "frac": round(proj_bytes[k] / (v * 1e-3) / 1e9 / (HBM_PEAK_TBS * 1e3), 4)}
            for k, v in extra.items()}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
