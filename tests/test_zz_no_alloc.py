"""rnn_igemm_noalloc (no counterpart in the reference; for callers that cannot
allocate): the igemm contract of src/int8.rs:285-314 with the workspace in the
library's file-scope device array. Checked bit for bit against rnn_igemm with
a caller-supplied workspace and against the oracle's scalar igemm
(src/int8.rs:222-234), on consecutive calls of different sizes -- the second
smaller than the first -- so a stale workspace from the previous call would
show."""
import ctypes

import numpy as np
import pytest

import oracle as O
import rnn_hip as H


def _case(m, k, n, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    a = g.integers(0, 256, size=(m, k), dtype=np.uint8)
    b = g.integers(-128, 128, size=(k, n), dtype=np.int8)
    return a, b


@pytest.mark.gpu
def test_igemm_noalloc_matches_igemm_on_consecutive_calls(dev, hip):
    import torch
    # (m n k above 2^28 runs on the array: the tiled path (m > 16), then a
    # smaller tiled call, then the GEMV path (m <= 16, k not a multiple of
    # 64); a small problem last, which takes the one-launch kernel and no
    # workspace)
    for m, k, n, seed in ((600, 1000, 640, 1), (400, 900, 800, 2), (12, 3000, 8000, 3),
                          (5, 70, 33, 4)):
        a, b = _case(m, k, n, seed)
        da, db = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
        ws = torch.empty(hip.igemm_workspace_size(m, k, n), dtype=torch.uint8, device=dev)
        ref = hip.igemm(da, db, m, k, n, workspace=ws)
        c = torch.full((m, n), -7, dtype=torch.int32, device=dev)   # no stale zeros to hide behind
        hip.igemm_noalloc(da, db, m, k, n, c)
        torch.cuda.synchronize()
        got = c.cpu().numpy()
        np.testing.assert_array_equal(got, ref.cpu().numpy())
        np.testing.assert_array_equal(got, O.igemm_scalar(a, b, m, k, n))


@pytest.mark.gpu
def test_igemm_noalloc_empty_reduction_and_limit(dev, hip):
    import torch
    c = torch.full((3, 4), 9, dtype=torch.int32, device=dev)
    a = torch.empty((3, 0), dtype=torch.uint8, device=dev)
    b = torch.empty((0, 4), dtype=torch.int8, device=dev)
    hip.igemm_noalloc(a, b, 3, 0, 4, c)        # k = 0: C = 0
    assert c.cpu().numpy().tolist() == [[0] * 4] * 3


def test_igemm_noalloc_rejects_sizes_beyond_the_array():
    lib = H.load()
    fake = ctypes.c_void_p(256)   # never dereferenced: the size check comes first
    # 8192 x 8192 x 8192 needs 128 MiB of workspace, twice the array
    assert H.igemm_workspace_size(8192, 8192, 8192) > H.IGEMM_NOALLOC_MAX_BYTES
    rc = lib.rnn_igemm_noalloc(fake, fake, fake, 8192, 8192, 8192, None)
    assert rc == H.RNN_ERR_UNSUPPORTED
    assert "device array" in H.last_error()
    assert lib.rnn_igemm_noalloc(fake, fake, fake, -1, 4, 4, None) == H.RNN_ERR_INVALID_ARG
    # A one-launch problem uses no workspace: m = n = 1, k = 2^25 needs more
    # workspace than the array holds under the packed plan, yet is not refused
    # for it. Only where no GPU is present: the call then reaches the launch
    # and fails there with a HIP error (with a GPU the fake pointers would be
    # read; test_igemm_noalloc_small_problem_beyond_the_array runs it for real).
    import torch
    assert H.igemm_workspace_size(1, 2**25, 1) > H.IGEMM_NOALLOC_MAX_BYTES
    if torch.cuda.device_count() == 0:
        rc = lib.rnn_igemm_noalloc(fake, fake, fake, 1, 2**25, 1, None)
        assert rc == H.RNN_ERR_HIP, H.last_error()


@pytest.mark.gpu
def test_igemm_noalloc_small_problem_beyond_the_array(dev, hip):
    """m = n = 1, k = 2^25: m n k is within the one-launch bound, so no
    workspace is needed although the packed plan's would exceed the array."""
    import torch
    k = 2**25
    g = np.random.default_rng(5)
    a = g.integers(0, 256, size=(1, k), dtype=np.uint8)
    b = g.integers(-128, 128, size=(k, 1), dtype=np.int8)
    c = torch.full((1, 1), 7, dtype=torch.int32, device=dev)
    hip.igemm_noalloc(torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev), 1, k, 1, c)
    exact = int((a.astype(np.int64) @ b.astype(np.int64))[0, 0])
    want = (exact + 2**31) % 2**32 - 2**31   # wrapping int32
    assert int(c.cpu().numpy()[0, 0]) == want
