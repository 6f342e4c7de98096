"""The plain-read helper behind bench.py's stream_floor_us (libqr_floor.so, not part of the
attention library): it loads, exports its one entry point, and rejects invalid arguments
before any device call; on the GPU a read of a few sets returns 0 and leaves its input
unchanged."""
import ctypes
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PATH = os.path.join(ROOT, "qauntrunner_amd", "libqr_floor.so")


def load():
    lib = ctypes.CDLL(PATH)
    lib.qr_floor_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                  ctypes.c_int, ctypes.c_void_p]
    lib.qr_floor_read.restype = ctypes.c_int
    return lib


@pytest.mark.parametrize("buf,nbytes,sets,reps,sink,blocks", [
    (None, 4096, 1, 1, 64, 256),      # no buffer
    (4096, 4096, 1, 1, None, 256),    # no sink
    (4096, 8, 1, 1, 64, 256),         # fewer than 16 bytes
    (4096, 4100, 1, 1, 64, 256),      # not a multiple of 16
    (4096, 4096, 0, 1, 64, 256),      # no sets
    (4096, 4096, 1, 0, 64, 256),      # no reads
    (4096, 4096, 1, 1, 64, 0),        # no workgroups
    (4096, 4096, 1, 1, 64, 70000),    # more workgroups than a grid dimension takes
    (4104, 4096, 1, 1, 64, 256),      # buffer not 16-byte aligned
])
def test_invalid_arguments_rejected_before_any_launch(buf, nbytes, sets, reps, sink, blocks):
    # the pointers are never dereferenced on these paths: the argument check comes first
    assert load().qr_floor_read(buf, nbytes, sets, reps, sink, blocks, None) == 1


@pytest.mark.gpu
def test_reads_return_and_leave_input_unchanged(gpu):
    import torch

    print("case: qr_floor_read over 3 sets of 1 MiB, 5 reads, 256 and 512 workgroups", flush=True)
    lib = load()
    n = 1 << 20
    buf = torch.arange(3 * n // 4, dtype=torch.int32, device=gpu)
    ref = buf.clone()
    sink = torch.zeros(64, dtype=torch.int32, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    for blocks in (256, 512):
        assert lib.qr_floor_read(buf.data_ptr(), n, 3, 5, sink.data_ptr(), blocks, stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(buf, ref)
