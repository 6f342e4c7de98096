"""Committed fixtures (tests/golden/, written by make_golden.py): the oracle must keep
reproducing them bit for bit, and the GPU path must match them within tolerance."""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle
from tests.util import assert_close

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_kat_fixture_matches_oracle_codecs():
    kats = json.load(open(os.path.join(HERE, "kats.json")))
    L = oracle.lib()
    for bits, want in kats["f16_to_f32"].items():
        got = L.qro_f16_to_f32(int(bits, 16))
        if want == "inf":
            assert math.isinf(got) and got > 0
        else:
            assert got == want and math.copysign(1, got) == math.copysign(1, want)
    for v in kats["bf16_round_trip_exact"]:
        assert L.qro_bf16_to_f32(L.qro_f32_to_bf16(v)) == v


def test_c1_fixture_reproduced_by_oracle():
    z = np.load(os.path.join(HERE, "c1_decode.npz"))
    H, HKV, D, _ = (int(x) for x in z["shape"])
    out = oracle.kv_attention(z["K"], z["V"], z["q"], H, HKV, D, float(z["scale"]))
    assert np.array_equal(out, z["out"])
    assert_close(out, z["out_f64"], 1e-5, 1e-5, "fixture oracle vs fp64")


def test_mla_fixture_reproduced_by_oracle():
    z = np.load(os.path.join(HERE, "mla_small.npz"))
    heads, lora, rope, _ = (int(x) for x in z["shape"])
    u = oracle.mla_attention(z["lat"], z["q_tilde"], z["q_rope"], lora, rope, float(z["scale"]))
    assert np.array_equal(u, z["u"])


@pytest.mark.gpu
def test_c1_fixture_on_gpu(gpu):
    import qauntrunner_amd as qr

    z = np.load(os.path.join(HERE, "c1_decode.npz"))
    H, HKV, D, SEQ = (int(x) for x in z["shape"])
    with qr.PagedKvCache(1, H, HKV, D, SEQ) as kv:
        kv.AppendRange(0, 0, z["K"], z["V"])
        got = kv.Attention(0, SEQ - 1, z["q"], float(z["scale"]))
    assert_close(got, z["out"], 1e-3, 1e-4, "C1 fixture")


@pytest.mark.gpu
def test_mla_fixture_on_gpu(gpu):
    import qauntrunner_amd as qr

    z = np.load(os.path.join(HERE, "mla_small.npz"))
    heads, lora, rope, seq = (int(x) for x in z["shape"])
    with qr.MlaLatentCache(1, lora + rope, seq, rope=rope) as m:
        m.AppendRange(0, 0, z["lat"])
        got = m.AbsorbedAttention(0, seq - 1, z["q_tilde"], z["q_rope"], float(z["scale"]))
    assert_close(got, z["u"], 1e-3, 1e-4, "MLA fixture (fp32 latents)")
