"""Writes the committed fixtures under tests/golden/.

* kats.json: the known-answer constants of the reference's dtype tests
  (tests/QuantRunner.Tests/Program.cs:60-92) as data.
* c1_decode.npz: the 8-head / 2-kv-head / head_dim 64 / 512-token decode case
  (seeded N(0,1) inputs) with the oracle's output and the fp64 output.
* mla_small.npz: an 8-head MLA absorbed case (kv_lora 512, rope 64, 260 tokens).

Run: python tests/golden/make_golden.py   (CPU only; regenerates byte-identical files)
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle  # noqa: E402


def main():
    kats = {
        "f16_to_f32": {"0x0000": 0.0, "0x8000": -0.0, "0x3c00": 1.0, "0xbc00": -1.0, "0x7bff": 65504.0,
                       "0x7c00": "inf", "0x0001": 2.0 ** -24},
        "f16_round_trip_rel_tol_normal": 0.0005,
        "f16_round_trip_abs_tol_subnormal": 6e-08,
        "bf16_round_trip_exact": [1.0, -2.5],
        "bf16_pi_rel_tol": 0.01,
    }
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1, sort_keys=True)

    rng = np.random.default_rng(20261201)
    H, HKV, D, SEQ = 8, 2, 64, 512
    q = rng.standard_normal(H * D, dtype=np.float32)
    K = rng.standard_normal((SEQ, HKV * D), dtype=np.float32)
    V = rng.standard_normal((SEQ, HKV * D), dtype=np.float32)
    out = oracle.kv_attention(K, V, q, H, HKV, D, 0.125)
    out64 = oracle.kv_attention_f64(K, V, q, H, HKV, D, 0.125)
    np.savez(os.path.join(HERE, "c1_decode.npz"), q=q, K=K, V=V, scale=np.float32(0.125),
             shape=np.array([H, HKV, D, SEQ], np.int32), out=out, out_f64=out64)

    rng = np.random.default_rng(20261202)
    heads, lora, rope, seq = 8, 512, 64, 260
    lat = rng.standard_normal((seq, lora + rope), dtype=np.float32)
    qt = rng.standard_normal((heads, lora), dtype=np.float32)
    qr = rng.standard_normal((heads, rope), dtype=np.float32)
    s = np.float32(1 / np.sqrt(192.0))
    u = oracle.mla_attention(lat, qt, qr, lora, rope, float(s))
    u64 = oracle.mla_attention_f64(lat, qt, qr, lora, rope, float(s))
    np.savez(os.path.join(HERE, "mla_small.npz"), lat=lat, q_tilde=qt, q_rope=qr, scale=s,
             shape=np.array([heads, lora, rope, seq], np.int32), u=u, u_f64=u64)


if __name__ == "__main__":
    main()
