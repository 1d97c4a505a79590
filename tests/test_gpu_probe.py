"""The benchmark's read-floor helper (librnn_probe.so, rnn_probe_read): it must
read every byte it is given, or the floor it times would be too fast. One
planted 16-byte word in an otherwise zero buffer makes exactly one block's XOR
equal the magic value, and only then is the sink written; the cases put it at
the start, in the middle and in the last chunk, including a ragged last
block."""
import ctypes
import os

import numpy as np
import pytest

import rnn_hip as H

pytestmark = pytest.mark.gpu
PROBE = os.path.join(os.path.dirname(H.LIB_PATH), "librnn_probe.so")


@pytest.mark.parametrize("nbytes,where,per", [(1 << 20, 0, 16), (1 << 20, (1 << 20) - 16, 8),
                                              (45 * 2**20 + 4096, 12345 * 16, 32),
                                              (3 * 2**20 + 48, 3 * 2**20 + 32, 4)])
def test_read_floor_reads_every_chunk(dev, nbytes, where, per):
    import torch
    lib = ctypes.CDLL(PROBE)
    lib.rnn_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint32,
                                   ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    magic = 0x5EED1234
    buf[where // 4] = magic
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.rnn_probe_read(ctypes.c_void_p(buf.data_ptr()), nbytes, magic,
                              ctypes.c_void_p(sink.data_ptr()), per, ctypes.c_void_p(st)) == 0
    assert int(sink.item()) == magic
    assert lib.rnn_probe_read(ctypes.c_void_p(buf.data_ptr()), 20, magic,
                              ctypes.c_void_p(sink.data_ptr()), 16, ctypes.c_void_p(st)) == 1
    assert lib.rnn_probe_read(ctypes.c_void_p(buf.data_ptr()), 64, magic,
                              ctypes.c_void_p(sink.data_ptr()), 3, ctypes.c_void_p(st)) == 1
