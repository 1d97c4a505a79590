"""The benchmark's read helpers (librnn_probe.so: rnn_probe_read, the read
floor, rnn_probe_range_read, the one-workgroup-per-share read, and
rnn_probe_l2_rate, the per-CU load rate): each must read what it is given,
or the rate it times would be too high. One
planted 16-byte word in an otherwise zero buffer makes exactly one block's
(range read: one wave's) XOR equal the magic value, and only then is the sink
written; the cases put it at the start, in the middle and in the last chunk,
including a ragged last block."""
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


@pytest.mark.parametrize("nbytes,where,groups,waves,per",
                         [(1 << 20, 0, 256, 8, 4), (1 << 20, (1 << 20) - 16, 256, 4, 24),
                          (45088768, 22544384 + 48, 256, 8, 8), (300 * 1024, 299 * 1024 + 512, 7, 4, 2),
                          (64 * 1024, 33 * 1024, 64, 8, 24)])
def test_range_read_reads_every_chunk(dev, nbytes, where, groups, waves, per):
    """rnn_probe_range_read (one workgroup per share, a chosen load depth):
    the same planted-word check, with shares of one chunk, ragged shares
    (300 chunks over 7 workgroups) and a depth larger than a wave's part of
    its share."""
    import torch
    lib = ctypes.CDLL(PROBE)
    lib.rnn_probe_range_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
                                         ctypes.c_void_p, ctypes.c_void_p]
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    magic = 0x5EED4321
    buf[where // 4] = magic
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = ctypes.c_void_p(buf.data_ptr())
    assert lib.rnn_probe_range_read(p, nbytes, groups, waves, per, magic,
                                    ctypes.c_void_p(sink.data_ptr()), st) == 0
    assert int(sink.item()) == magic
    # bad arguments: a ragged byte count, fewer chunks than workgroups, an
    # unbuilt depth
    assert lib.rnn_probe_range_read(p, 1000, 1, 4, 4, magic, ctypes.c_void_p(sink.data_ptr()), st) == 1
    assert lib.rnn_probe_range_read(p, 4096, 8, 4, 4, magic, ctypes.c_void_p(sink.data_ptr()), st) == 1
    assert lib.rnn_probe_range_read(p, 4096, 1, 4, 3, magic, ctypes.c_void_p(sink.data_ptr()), st) == 1


@pytest.mark.parametrize("to_lds,per,window,chunk", [(0, 4, 5, 10), (0, 8, 13, 0), (1, 4, 9, 63),
                                                     (1, 8, 2, 60)])
def test_l2_rate_reads_what_it_times(dev, to_lds, per, window, chunk):
    """rnn_probe_l2_rate: 2 blocks of 8 waves over 16 windows of 64 KiB, one
    window per wave, 64 / per rounds: VGPR loads XOR every chunk of the
    window once; LDS loads leave the last round's chunks (60..63 at 4 per
    round, 56..63 at 8) in LDS. One planted word makes that wave's XOR the
    magic value; bad arguments return 1."""
    import torch
    lib = ctypes.CDLL(PROBE)
    lib.rnn_probe_l2_rate.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_uint32,
                                      ctypes.c_void_p, ctypes.c_void_p]
    nbytes = 16 << 16
    buf = torch.zeros(nbytes // 4, dtype=torch.int32, device=dev)
    magic = 0x5EED6789
    buf[(window * 65536 + chunk * 1024 + 16 * 7) // 4] = magic
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = ctypes.c_void_p(buf.data_ptr())
    assert lib.rnn_probe_l2_rate(p, nbytes, 2, to_lds, per, 64 // per, magic,
                                 ctypes.c_void_p(sink.data_ptr()), st) == 0
    assert int(sink.item()) == magic
    bad = dict(bytes=nbytes, groups=2, lds=to_lds, per=per)
    for k, v in (("bytes", 65536 + 16), ("groups", 0), ("lds", 2), ("per", 3)):
        a = dict(bad, **{k: v})
        assert lib.rnn_probe_l2_rate(p, a["bytes"], a["groups"], a["lds"], a["per"], 4, magic,
                                     ctypes.c_void_p(sink.data_ptr()), st) == 1

