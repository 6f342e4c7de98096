"""A process that exits with library handles still open on the GPU ends with status 0.

The handles (a paged K/V cache, an MLA latent cache, a resident weight) are closed by the
library's atexit hook while the HIP runtime is still whole; the Python finalizers that run
later, during interpreter shutdown, do nothing.  The child process runs one attention call on
each cache first, so every handle holds device buffers when the process ends.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = """
import sys
sys.path.insert(0, %r)
import numpy as np
import torch
import qauntrunner_amd as qr
dev = torch.device("cuda:0")
rng = np.random.default_rng(5)
kv = qr.PagedKvCache(1, 8, 2, 128, 1024, kv_dtype="f16")
k = torch.from_numpy(rng.standard_normal((600, 256), dtype=np.float32)).to(dev)
kv.AppendRangeDev(0, 0, k, k)
q = torch.from_numpy(rng.standard_normal(8 * 128, dtype=np.float32)).to(dev)
out = torch.empty(8 * 128, device=dev)
kv.AttentionDev(0, [0], [599], q, out, 0.088)
m = qr.MlaLatentCache(1, 576, 512, dtype="bf16", rope=64)
m.AppendRange(0, 0, rng.standard_normal((300, 576), dtype=np.float32))
u = m.AbsorbedAttention(0, 299, rng.standard_normal((16, 512), dtype=np.float32),
                        rng.standard_normal((16, 64), dtype=np.float32), 0.07)
w = qr.Weight("F32", 64, 256, rng.standard_normal((64, 256), dtype=np.float32).view(np.uint8))
y = w.MatVec(np.ones(256, np.float32))
torch.cuda.synchronize()
keep = [kv, m, w]  # still referenced when the interpreter finalizes
print("ok", float(out.abs().sum().item()) > 0, bool(np.isfinite(u).all()), bool(np.isfinite(y).all()))
sys.stdout.flush()
"""


def test_exit_with_open_gpu_handles(gpu):
    print("case: child process exits with open K/V, MLA and weight handles", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD % ROOT], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-4000:])
    assert r.stdout.split() == ["ok", "True", "True", "True"], r.stdout
