"""Synthetic .qw models for the ModelStore / PrefetchPipeline tests.

The tensor list follows the reference's synthetic test model (SynthShared.WriteModel,
tests/QuantRunner.Tests/Program.cs:551-630): tok_emb and lm_head in F16, F32 norms, and
per layer wq/wk/wv/wo plus either a dense FFN or a router and per-expert FFNs.  Weights
are seeded normal values encoded by tests.quant; the bytes each tensor holds are
returned so the tests can compare against the oracle on exactly those bytes.
"""
from __future__ import annotations

import numpy as np

from qauntrunner_amd.store import ModelStoreBuilder
from tests import quant


def plan(dim=256, layers=3, heads=4, ffn=512, vocab=256, experts=0, fmt="Q4_K"):
    """(name, dims, format name) in the reference's plan order."""
    head_dim = dim // heads
    out = [("tok_emb", (vocab, dim), "F16"), ("final_norm", (dim,), "F32")]
    for l in range(layers):
        out += [(f"l{l}.attn_norm", (dim,), "F32"), (f"l{l}.wq", (dim, dim), fmt),
                (f"l{l}.wk", (heads * head_dim, dim), fmt), (f"l{l}.wv", (heads * head_dim, dim), fmt),
                (f"l{l}.wo", (dim, dim), fmt), (f"l{l}.ffn_norm", (dim,), "F32")]
        if experts:
            out.append((f"l{l}.router", (experts, dim), "F32"))
            for e in range(experts):
                out += [(f"l{l}.e{e}.w_gate", (ffn, dim), fmt), (f"l{l}.e{e}.w_up", (ffn, dim), fmt),
                        (f"l{l}.e{e}.w_down", (dim, ffn), fmt)]
        else:
            out += [(f"l{l}.w_gate", (ffn, dim), fmt), (f"l{l}.w_up", (ffn, dim), fmt),
                    (f"l{l}.w_down", (dim, ffn), fmt)]
    out.append(("lm_head", (vocab, dim), "F16"))
    return out


def write(path, seed=8, header_reserve_bytes=0, **kw):
    """Writes the model; returns {name: (format code, dims, uint8 bytes)}."""
    tensors = {}
    for i, (name, dims, fmt) in enumerate(plan(**kw)):
        code = quant.FMT[fmt]
        rows = int(np.prod(dims[:-1])) if len(dims) > 1 else 1
        raw, _ = quant.random_rows(code, rows, dims[-1], seed * 1000 + i, std=0.02)
        tensors[name] = (code, tuple(dims), np.ascontiguousarray(raw).reshape(-1))
    b = ModelStoreBuilder(path, {"arch": "moe" if kw.get("experts") else "llama", "dim": kw.get("dim", 256),
                                 "layers": kw.get("layers", 3)}, header_reserve_bytes)
    for name, (code, dims, raw) in tensors.items():
        b.Plan(name, dims, code, raw.size)
    b.Commit(lambda name: tensors[name][2])
    return tensors


def layer_bytes(tensors, layer):
    """Bytes the pipeline stages for `layer`: its tensors minus names ending in norm/router."""
    pre = "" if layer < 0 else f"l{layer}."
    return sum(t[2].size for n, t in tensors.items()
               if n.startswith(pre) and not n.endswith("norm") and not n.endswith("router"))
