"""GPU parity of rnn_sgemm (the BlasBackend::sgemm plugin point,
src/blas.rs:712-734) against the oracle's restatement of the reference's
contract. f32 products are accumulated with fused multiply-adds in the
kernel's own order, so the bar is the GEMM rounding bound
|got - exact| <= gamma_(k+2) * (|alpha| |A||B| + |beta C|) (gamma_j = j u /
(1 - j u), u = 2^-24) around the float64 value, plus the reference's own test
tolerances; the special cases of the contract (beta = 0 overwrites, k = 0 or
alpha = 0 scales, untouched padding) are exact."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def bound(k, scale):
    u = 2.0 ** -24
    return (k + 2) * u / (1 - (k + 2) * u) * scale + 1e-30


def run(dev, hip, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, ldc):
    c = to_dev(c0, dev)
    hip.sgemm(ta, tb, m, n, k, alpha, to_dev(a, dev), lda, to_dev(b, dev), ldb, beta, c, ldc)
    return c.cpu().numpy()


def check(got_flat, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, ldc):
    exact, scale = O.sgemm_f64(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, ldc)
    got = np.lib.stride_tricks.as_strided(got_flat, shape=(m, n), strides=(ldc * 4, 4))
    err = np.abs(got.astype(np.float64) - exact)
    lim = bound(k, scale)
    assert np.all(err <= lim), f"max err {err.max():.3g}, worst excess {(err - lim).max():.3g}"
    # padding columns of C (ldc > n) untouched
    if ldc > n:
        pad = np.lib.stride_tricks.as_strided(got_flat[n:], shape=(m - 1, ldc - n), strides=(ldc * 4, 4))
        pad0 = np.lib.stride_tricks.as_strided(np.asarray(c0, np.float32)[n:], shape=(m - 1, ldc - n),
                                               strides=(ldc * 4, 4))
        assert np.array_equal(pad, pad0)


@pytest.mark.parametrize("case", O.BLAS_TEST_CASES, ids=[c[0] for c in O.BLAS_TEST_CASES])
def test_sgemm_reference_cases(dev, hip, case):
    """The reference's sgemm tests (src/blas.rs:1195-1470) through the C ABI,
    against the oracle within the reference's tolerance and the rounding
    bound."""
    _, ta, tb, m, n, k, seed, alpha, beta, tol = case
    a, lda, b, ldb, c0 = O.blas_test_case(ta, tb, m, n, k, seed, beta)
    got = run(dev, hip, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, n)
    ref = O.sgemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, n)
    assert np.abs(got - ref).max() < tol
    check(got, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, n)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k,alpha,beta,pad", [
    (128, 128, 128, 1.0, 0.0, 0),        # one block tile, MFMA path
    (130, 260, 300, 0.5, 2.0, 0),        # ragged edges in m and n, K tail (MFMA path)
    (32, 256, 784, 1.0, 0.0, 0),         # config-1 MLP layer shape
    (517, 301, 95, -1.25, 1.0, 3),       # odd k and padded strides -> one-thread-per-output path
    (256, 384, 1024, 1.0, -0.5, 4),      # padded strides (MFMA path; 6 tiles: K split in 4)
    (64, 1000, 4128, 1.5, 0.5, 0),       # 8 tiles: K split in 15 ranges, the last one short
    (16, 300, 784, 1.0, 0.5, 0),         # transb: the skinny kernel, a K tail, 19 row tiles
    (5, 4100, 1056, -1.0, 0.0, 4),       # transb: skinny, padded strides, a ragged last tile
    (3, 8200, 64, 2.0, 1.0, 0),          # transb: skinny, 2 tiles per workgroup, 2 of 4 waves idle
    (7, 260, 4096, 0.5, 0.0, 0),         # transb: skinny, 32 steps per wave (the steady loop)
    (16, 8200, 2056, 1.0, 0.5, 0),       # B as stored: skinny NN, K tail, ragged last block
    (9, 300, 100, 2.0, 0.0, 8),          # B as stored: skinny NN, short K, padded strides
])
def test_sgemm_shapes(dev, hip, ta, tb, m, n, k, alpha, beta, pad):
    rng = np.random.default_rng(m * 7 + n * 3 + k + 11 * ta + 13 * tb)
    ra, ca = (k, m) if ta else (m, k)
    rb, cb = (n, k) if tb else (k, n)
    lda, ldb, ldc = ca + pad, cb + pad, n + pad
    a = rng.standard_normal(ra * lda).astype(np.float32)
    b = rng.standard_normal(rb * ldb).astype(np.float32)
    c0 = rng.standard_normal(m * ldc).astype(np.float32)
    got = run(dev, hip, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, ldc)
    check(got, ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, ldc)


def test_sgemm_contract_special_cases(dev, hip):
    # matmul_convenience_works (src/blas.rs:1514-1520), through matmul()
    import torch
    c = hip.matmul(to_dev(np.array([[1, 2], [3, 4]]), dev), to_dev(np.array([[5, 6], [7, 8]]), dev))
    assert c.cpu().numpy().tolist() == [[19.0, 22.0], [43.0, 50.0]]
    # beta = 0 overwrites C without reading it: NaN in C does not propagate
    m = n = k = 64
    a = np.ones(m * k, np.float32)
    nan_c = np.full(m * n, np.nan, np.float32)
    got = run(dev, hip, 0, 0, m, n, k, 1.0, a, k, a, n, 0.0, nan_c, n)
    assert np.all(got == 64.0)
    # k = 0: C = beta*C (beta = 0 -> zeros, even over NaN); alpha = 0 likewise
    assert np.all(run(dev, hip, 0, 0, m, n, 0, 1.0, a, 1, a, n, 0.0, nan_c, n) == 0.0)
    c0 = np.arange(m * n, dtype=np.float32)
    assert np.array_equal(run(dev, hip, 0, 0, m, n, k, 0.0, a, k, a, n, 2.0, c0, n), 2.0 * c0)
    assert np.array_equal(run(dev, hip, 1, 1, m, n, 0, 3.0, a, m, a, 1, 1.0, c0, n), c0)
    # the HipBackend mirror of the trait
    be = hip.HipBackend()
    assert "hip" in be.name()
    cd = to_dev(np.zeros(4), dev)
    be.sgemm(hip.NO_TRANS, hip.NO_TRANS, 1, 1, 1, 1.0, to_dev([3.0], dev), 1, to_dev([4.0], dev), 1,
             0.0, cd, 1)
    assert cd.cpu().numpy()[0] == 12.0
    del torch


def test_sgemm_large_against_float64(dev, hip):
    """2048 x 2048 x 2048 on the MFMA path, every output, against a float64
    product on the device, within the rounding bound."""
    import torch
    m = n = k = 2048
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    a = torch.randn((m, k), generator=g, device=dev)
    b = torch.randn((k, n), generator=g, device=dev)
    c = torch.empty((m, n), device=dev)
    hip.sgemm(hip.NO_TRANS, hip.NO_TRANS, m, n, k, 1.0, a, k, b, n, 0.0, c, n)
    exact = a.double() @ b.double()
    scale = a.double().abs() @ b.double().abs()
    u = 2.0 ** -24
    lim = (k + 2) * u / (1 - (k + 2) * u) * scale
    assert bool(((c.double() - exact).abs() <= lim).all())


def test_sgemm_split_and_skinny_repeatable(dev, hip):
    """The split-K route (fewer tiles than CUs: partial tiles in scratch, summed
    in a fixed order) and the skinny m <= 16 kernels for both B layouts
    (waves' partial tiles summed in wave order) give the same bits on every
    call, and agree with a float64 product within the rounding bound."""
    rng = np.random.default_rng(77)
    for (m, n, k, tb) in ((64, 1000, 4128, 0), (64, 1000, 4128, 1), (16, 2000, 4096, 1),
                          (16, 2000, 4096, 0)):
        a = rng.standard_normal(m * k).astype(np.float32)
        b = rng.standard_normal(n * k).astype(np.float32)
        ldb = k if tb else n
        c0 = np.zeros(m * n, np.float32)
        runs = [run(dev, hip, 0, tb, m, n, k, 1.0, a, k, b, ldb, 0.0, c0, n) for _ in range(3)]
        assert all(np.array_equal(runs[0].view(np.uint32), r.view(np.uint32)) for r in runs[1:])
        check(runs[0], 0, tb, m, n, k, 1.0, a, k, b, ldb, 0.0, c0, n)


def test_sgemm_nn_through_transposed_b(dev, hip):
    """C = A B with B as stored and at least 2048 rows: B is transposed into
    scratch (64 x 64 tiles, ragged here in both N and K) and the product runs
    on the both-K-contiguous kernel; padded strides, alpha and beta, within
    the rounding bound, padding columns of C untouched."""
    rng = np.random.default_rng(2052)
    m, n, k, pad = 2048, 2052, 1056, 4
    lda, ldb, ldc = k + pad, n + pad, n + pad
    a = rng.standard_normal(m * lda).astype(np.float32)
    b = rng.standard_normal(k * ldb).astype(np.float32)
    c0 = rng.standard_normal(m * ldc).astype(np.float32)
    got = run(dev, hip, 0, 0, m, n, k, 0.75, a, lda, b, ldb, -0.5, c0, ldc)
    check(got, 0, 0, m, n, k, 0.75, a, lda, b, ldb, -0.5, c0, ldc)
