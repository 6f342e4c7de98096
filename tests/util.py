"""Shared helpers of the tests: seeded inputs and error metrics."""
from __future__ import annotations

import numpy as np

from oracle import oracle


def normal(seed, shape):
    """i.i.d. N(0,1) fp32 from a seeded PCG64 stream."""
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def to_dtype_bits(x, dtype):
    """fp32 -> (storage array, exactly decoded fp32 values) for a cache dtype.
    16-bit values are rounded once (RNE, numpy's conversion for fp16; the
    reference codec for bf16) and both sides receive the same bit patterns."""
    if dtype == "f32":
        return x, x
    if dtype == "f16":
        bits = x.astype(np.float16).view(np.uint16)
        return bits, oracle.f16_to_f32(bits)
    bits = oracle.f32_to_bf16(x)
    return bits, oracle.bf16_to_f32(bits)


def errors(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    max_abs = float(np.max(np.abs(got - want))) if got.size else 0.0
    rel = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))
    return max_abs, rel


def assert_close(got, want, max_abs, rel_l2, what=""):
    a, r = errors(got, want)
    assert a <= max_abs and r <= rel_l2, f"{what}: max-abs {a:.3e} (<= {max_abs}), rel-L2 {r:.3e} (<= {rel_l2})"
    return a, r
