"""The benchmark's streaming-read probe (measure/libalveare_probe.so, a
measurement aid outside the product library): it reads every byte of the
buffer, at every launch shape the benchmark sweeps."""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_stream_read_probe(dev):
    path = os.path.join(ROOT, "measure", "libalveare_probe.so")
    assert os.path.exists(path), "measure/libalveare_probe.so is not built"
    L = ctypes.CDLL(path)
    L.alvprobe_stream_read.restype = ctypes.c_int
    L.alvprobe_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_void_p]
    L.alvprobe_last_error.restype = ctypes.c_char_p
    st = torch.cuda.current_stream().cuda_stream
    for n in (4, 1 << 20, (1 << 20) + 12):  # words: one chunk, 4 MiB, a ragged tail
        buf = torch.randint(-2**31, 2**31 - 1, (n,), dtype=torch.int32, device=dev)
        sink = torch.zeros(2048, dtype=torch.int32, device=dev)
        want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
        for wg, depth in ((4, 4), (1, 2), (2, 16), (8, 8), (3, 4)):
            sink.zero_()
            assert L.alvprobe_stream_read(buf.data_ptr(), n * 4, sink.data_ptr(), wg, depth, st) == 0
            assert np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32)[::32]) == want, (n, wg, depth)
    assert L.alvprobe_stream_read(buf.data_ptr(), 16, sink.data_ptr(), 4, 3, st) != 0
    assert b"read shape" in L.alvprobe_last_error()
    assert L.alvprobe_stream_read(buf.data_ptr(), 16, sink.data_ptr(), 9, 4, st) != 0
