"""GPU parity: int8 quantization, igemm and W8A8 GEMM/GEMV through the C ABI
against the CPU oracle. int32 accumulators and int8 codes must be bit-exact;
fp32 outputs are required bit-exact too (same expressions, no contraction),
which is stricter than the 1e-5 relative contract."""
import numpy as np
import pytest

import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5  # the contract; the assertions below demand exact equality


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.cpu().numpy()


def assert_f32_equal(got, exp):
    assert got.shape == exp.shape
    bad = ~((got == exp) | (np.isnan(got) & np.isnan(exp)))
    if bad.any():
        i = np.argwhere(bad)[0]
        rel = np.abs(got[bad] - exp[bad]) / np.maximum(np.abs(exp[bad]), 1e-30)
        raise AssertionError(f"{bad.sum()} mismatches, first at {i}: {got[tuple(i)]} vs "
                             f"{exp[tuple(i)]}; max rel {rel.max():.3g} (contract {REL_TOL})")


# ------------------------------------------------------------------ quantization
@pytest.mark.parametrize("rows,cols", [(1, 4096), (16, 4096), (33, 784), (7, 13), (5, 1), (3, 0),
                                       (2048, 4096)])
def test_quant_rows_i8_parity(dev, hip, rows, cols):
    x = W.activations(rows, cols, seed=rows * 7 + cols, outlier_frac=0.01)
    if rows > 2:
        x[1] = 0.0
        x[2, : min(cols, 3)] = np.float32(2.5) * np.float32(1e-3)
    q, s = hip.quant_rows_i8(to_dev(x, dev))
    qo, so = O.quant_rows_i8(x)
    assert np.array_equal(host(s), so)
    assert np.array_equal(host(q), qo)


@pytest.mark.parametrize("cols", [4, 1020, 1024, 2048, 3000, 4096, 8192, 8196])
def test_quant_rows_register_path_edges(dev, hip, cols):
    """The register-resident quantizer (cols % 4 == 0 up to 8192; the strided
    kernel past it) against the oracle: exact half-integer quotients (where
    round() and a rounded reciprocal product could disagree), NaN and +-inf
    in aligned rows, a zero row, a subnormal-only row, and ordinary rows."""
    g = np.random.Generator(np.random.PCG64(cols))
    x = g.standard_normal((8, cols), dtype=np.float32)
    # row 0: scale 0.25 (max 31.75), every other value an exact (k + 0.5) * 0.25
    k = g.integers(-127, 127, size=cols).astype(np.float32)
    x[0] = (k + np.float32(0.5)) * np.float32(0.25)
    x[0, 0] = np.float32(31.75)
    # row 1: the same with a scale that is not a power of two (half quotients
    # are then whatever m / 127 makes of them: the division decides)
    x[1] = x[0] * np.float32(1.3)
    x[2, cols // 2] = np.nan
    x[3, 0] = np.inf
    x[4, -1] = -np.inf
    x[5] = 0.0
    x[6] = g.standard_normal(cols).astype(np.float32) * np.float32(1e-39)   # subnormal
    q, s = hip.quant_rows_i8(to_dev(x, dev))
    qo, so = O.quant_rows_i8(x)
    assert np.array_equal(host(s), so, equal_nan=True)
    assert np.array_equal(host(q), qo)


def test_quant_rows_nan_and_unaligned(dev, hip):
    import torch
    x = W.activations(4, 33, seed=1)
    x[0, 5] = np.nan
    buf = to_dev(np.concatenate([np.zeros(1, np.float32), x.ravel()]), dev)
    xv = buf[1:].view(4, 33)  # 4-byte aligned only: exercises the scalar path
    q = torch.empty((4, 33), dtype=torch.int8, device=dev)
    s = torch.empty(4, dtype=torch.float32, device=dev)
    hip.quant_rows_i8(xv, q, s)
    qo, so = O.quant_rows_i8(x)
    assert np.array_equal(host(s), so) and np.array_equal(host(q), qo)


def test_int8_dequantize_parity(dev, hip):
    w = W.weights(64, 200, seed=2)
    qo, so = O.quant_rows_i8(w)
    got = host(hip.int8_dequantize(to_dev(qo, dev), to_dev(so, dev)))
    assert np.array_equal(got, O.int8_dequantize(qo, so))


# ------------------------------------------------------------------ reference Int8Linear
@pytest.mark.parametrize("batch,in_f,out_f", [(2, 8, 4), (32, 784, 256), (3, 17, 300)])
def test_int8_linear_forward_parity(dev, hip, batch, in_f, out_f):
    w = W.weights(out_f, in_f, seed=in_f)
    x = W.activations(batch, in_f, seed=out_f) * np.float32(0.01)
    bias = W.activations(1, out_f, seed=3)[0]
    wq, ws = O.quant_rows_i8(w)
    got = host(hip.int8_linear_forward(to_dev(x, dev), to_dev(wq, dev), to_dev(ws, dev),
                                       to_dev(bias, dev)))
    assert_f32_equal(got, O.int8_linear_forward(x, wq, ws, bias))
    got = host(hip.int8_linear_forward(to_dev(x, dev), to_dev(wq, dev), to_dev(ws, dev)))
    assert_f32_equal(got, O.int8_linear_forward(x, wq, ws))


def test_int8_matmul_f32_parity(dev, hip):
    w = W.weights(50, 96, seed=4)
    x = W.activations(6, 96, seed=5) * np.float32(0.02)
    wq, ws = O.quant_rows_i8(w)
    got = host(hip.int8_matmul_f32(to_dev(wq, dev), to_dev(ws, dev), to_dev(x, dev)))
    assert_f32_equal(got, O.int8_matmul_f32(wq, ws, x))


# ------------------------------------------------------------------ igemm
def lcg_case(m, k, n):
    a, s = O.lcg_bytes(1, m * k, signed=False)
    b, _ = O.lcg_bytes(s, k * n, signed=True)
    return a.view(np.uint8).reshape(m, k), b.reshape(k, n)


def test_igemm_known_small(dev, hip):
    # src/int8.rs:416-422
    a = to_dev(np.array([[1, 2, 3, 4]], np.uint8), dev)
    b = to_dev(np.array([1, -1, 2, 2, -3, 4, 0, -2], np.int8).reshape(4, 2), dev)
    assert host(hip.igemm(a, b, 1, 4, 2)).ravel().tolist() == [-4, 7]


@pytest.mark.parametrize("shape", [(16, 32, 48), (3, 5, 7), (13, 17, 29), (1, 1, 1), (4, 4, 16),
                                   (33, 9, 33), (64, 64, 64)])
def test_igemm_lcg_shapes(dev, hip, shape):
    # src/int8.rs:425-433 (worst abs diff must be 0)
    m, k, n = shape
    a, b = lcg_case(m, k, n)
    got = host(hip.igemm(to_dev(a, dev), to_dev(b, dev), m, k, n))
    assert np.array_equal(got, O.igemm_scalar(a, b, m, k, n))


@pytest.mark.parametrize("m,k,n", [(512, 512, 512), (17, 300, 1000), (300, 4096, 129),
                                   (7, 2048, 300), (16, 4096, 5000),
                                   # m n k above 2^28: pack + transpose + column sums + the
                                   # 64 x 64 and the 128 x 128 tiled GEMMs
                                   (1024, 512, 1024), (2048, 128, 2048)])
def test_igemm_full_u8_range(dev, hip, m, k, n):
    # benches/core_ops.rs:152-153 inputs: a = i % 251 (u8), b = i % 255 (as i8)
    a = (np.arange(m * k) % 251).astype(np.uint8).reshape(m, k)
    b = (np.arange(k * n) % 255).astype(np.uint8).view(np.int8).reshape(k, n)
    import torch
    ws = torch.empty(hip.igemm_workspace_size(m, k, n), dtype=torch.uint8, device=dev)
    got = host(hip.igemm(to_dev(a, dev), to_dev(b, dev), m, k, n, workspace=ws))
    exp, _ = O.igemm(a, b, m, k, n, 8)
    assert np.array_equal(got, exp)


def test_igemm_small_unaligned_operands(dev, hip):
    """The one-launch kernel of small problems with a and b one byte past a
    16-byte boundary (byte loads instead of 16-byte ones), K over two 256-k
    chunks and a ragged last tile."""
    import torch
    m, k, n = 45, 300, 70
    a, b = lcg_case(m, k, n)
    ab = torch.zeros(m * k + 1, dtype=torch.uint8, device=dev)
    bb = torch.zeros(k * n + 1, dtype=torch.int8, device=dev)
    ab[1:] = torch.from_numpy(a.ravel()).to(dev)
    bb[1:] = torch.from_numpy(b.ravel()).to(dev)
    da, db = ab[1:].view(m, k), bb[1:].view(k, n)
    assert da.data_ptr() % 16 == 1 and db.data_ptr() % 16 == 1
    got = host(hip.igemm(da, db, m, k, n))
    assert np.array_equal(got, O.igemm_scalar(a, b, m, k, n))


def test_igemm_wrapping(dev, hip):
    m, k, n = 2, 70016, 3
    a = np.full((m, k), 255, np.uint8)
    b = np.full((k, n), 127, np.int8)
    got = host(hip.igemm(to_dev(a, dev), to_dev(b, dev), m, k, n))
    assert np.array_equal(got, O.igemm_scalar(a, b, m, k, n))


# ------------------------------------------------------------------ W8A8
def w8a8_case(m, k, n, seed, outliers=0.0):
    w = W.weights(n, k, seed=seed)
    x = W.activations(m, k, seed=seed + 1, outlier_frac=outliers)
    wq, sw = O.quant_rows_i8(w)
    aq, sa = O.quant_rows_i8(x)
    bias = W.activations(1, n, seed=seed + 2)[0] * np.float32(0.1)
    return aq, sa, wq, sw, bias


def run_w8a8(dev, hip, aq, sa, wq, sw, bias, relu, algo):
    y, acc = hip.w8a8_linear(to_dev(aq, dev), to_dev(sa, dev), to_dev(wq, dev), to_dev(sw, dev),
                             None if bias is None else to_dev(bias, dev), relu=relu, algo=algo,
                             want_acc=True)
    return host(y), host(acc)


@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (16, 64, 16), (5, 48, 37), (64, 256, 128),
                                   (130, 784, 257), (200, 1024, 300), (32, 784, 256), (32, 128, 10)])
@pytest.mark.parametrize("algo", ["auto", "tiled"])
def test_w8a8_small_shapes(dev, hip, m, k, n, algo):
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=m + k + n)
    a = hip.ALGO_AUTO if algo == "auto" else hip.ALGO_TILED
    for relu, b in ((False, None), (True, bias)):
        y, acc = run_w8a8(dev, hip, aq, sa, wq, sw, b, relu, a)
        ye, acce = O.w8a8_linear(aq, sa, wq, sw, b, relu)
        assert np.array_equal(acc, acce)
        assert_f32_equal(y, ye)


@pytest.mark.parametrize("m,k,n", [(17, 128, 4), (64, 256, 128), (129, 128, 228), (200, 1024, 300),
                                   (256, 256, 224), (300, 384, 1000), (513, 640, 452),
                                   (1000, 128, 14336 // 16)])
def test_w8a8_lds_dma_kernel(dev, hip, m, k, n):
    """The LDS-DMA pipelined kernel (forced), on both tile variants (128x128
    with 4 waves for m <= 128, 256x224 with 8 waves above) with ragged M/N edges, against the oracle: int32
    bit-exact, fp32 bit-exact, for y only / acc only / both, bias + ReLU."""
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=3 * m + k + n, outliers=0.01)
    ye, acce = O.w8a8_linear(aq, sa, wq, sw, bias, True)
    d = [to_dev(a, dev) for a in (aq, sa, wq, sw, bias)]
    y, acc = hip.w8a8_linear(*d, relu=True, algo=hip.ALGO_TILED_DMA, want_acc=True)
    assert np.array_equal(host(acc), acce)
    assert_f32_equal(host(y), ye)
    _, acc2 = hip.w8a8_linear(*d, relu=True, algo=hip.ALGO_TILED_DMA, want_y=False, want_acc=True)
    assert np.array_equal(host(acc2), acce)
    y3, _ = hip.w8a8_linear(d[0], d[1], d[2], d[3], None, relu=False, algo=hip.ALGO_TILED_DMA)
    assert_f32_equal(host(y3), O.w8a8_linear(aq, sa, wq, sw)[0])


def test_w8a8_lds_dma_rejects_unsupported(dev, hip):
    aq, sa, wq, sw, _ = w8a8_case(32, 192, 64, seed=5)   # k % 128 != 0
    d = [to_dev(a, dev) for a in (aq, sa, wq, sw)]
    with pytest.raises(hip.RnnError) as e:
        hip.w8a8_linear(*d, algo=hip.ALGO_TILED_DMA)
    assert e.value.status == hip.RNN_ERR_UNSUPPORTED
    y, _ = hip.w8a8_linear(*d)                             # AUTO falls back to the staged kernel
    assert_f32_equal(host(y), O.w8a8_linear(aq, sa, wq, sw)[0])


def test_w8a8_activations_over_4gib(dev, hip):
    """An activation matrix of more than 4 GiB: the 128-byte-row kernel
    addresses its DMA sources with 32-bit offsets, so this shape takes the
    64-bit-addressed LDS-DMA kernel. Rows on both sides of byte offset 2^32
    (row 2^20 at K = 4096), the first and the last, against the oracle."""
    import torch
    k, n = 4096, 228                      # ragged N tile
    m = (1 << 20) + 300                   # 4 GiB + 1.2 MB of int8 activations
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    aq = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    sa = torch.rand(m, device=dev, generator=g) + 0.5
    _, _, wq, sw, bias = w8a8_case(4, k, n, seed=12)
    y, _ = hip.w8a8_linear(aq, sa, to_dev(wq, dev), to_dev(sw, dev), to_dev(bias, dev), relu=True)
    rows = [0, 1, (1 << 20) - 1, 1 << 20, (1 << 20) + 1, m - 1]
    idx = torch.tensor(rows, device=dev)
    aq_s, sa_s, y_s = host(aq[idx]), host(sa[idx]), host(y[idx])
    del aq, y
    torch.cuda.empty_cache()
    ye, _ = O.w8a8_linear(aq_s, sa_s, wq, sw, bias, True)
    assert_f32_equal(y_s, ye)


@pytest.mark.parametrize("m,k,n", W.GEMV_SHAPES)
def test_w8a8_decode_gemv_full_size(dev, hip, m, k, n):
    # BASELINE decode config: 1% activation outliers x20
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=n + m, outliers=0.01)
    y, acc = run_w8a8(dev, hip, aq, sa, wq, sw, None, False, hip.ALGO_AUTO)
    ye, acce = O.w8a8_linear(aq, sa, wq, sw)
    assert np.array_equal(acc, acce)
    assert_f32_equal(y, ye)
    # the tiled kernel agrees with the GEMV bit for bit
    y2, acc2 = run_w8a8(dev, hip, aq, sa, wq, sw, None, False, hip.ALGO_TILED)
    assert np.array_equal(acc2, acc) and np.array_equal(y2, y)


@pytest.mark.parametrize("m,k,n", [(2, 4096, 100), (3, 8192, 37), (4, 4096, 16), (5, 4096, 50),
                                   (7, 8192, 200), (16, 12288, 33), (1, 12288, 4)])
def test_w8a8_gemv_whole_line_variants(dev, hip, m, k, n):
    """The whole-line GEMV (K % 4096 == 0): the LDS-staged activation path
    (M <= 4) and the direct one (M > 4) with rows past M zeroed, ragged N,
    several 1 KiB K chunks per wave (K = 8192, 12288), bias + ReLU, and the
    accumulator-only output (no scales) -- int32 and fp32 bit-exact against
    the oracle."""
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=7 * m + n, outliers=0.01)
    ye, acce = O.w8a8_linear(aq, sa, wq, sw, bias, True)
    d = [to_dev(a, dev) for a in (aq, sa, wq, sw, bias)]
    y, acc = hip.w8a8_linear(*d, relu=True, want_acc=True)
    assert np.array_equal(host(acc), acce)
    assert_f32_equal(host(y), ye)
    _, acc2 = hip.w8a8_linear(d[0], None, d[2], None, None, want_y=False, want_acc=True)
    assert np.array_equal(host(acc2), acce)


@pytest.mark.parametrize("m,k,n", [(1, 4096, 4100), (3, 2048, 11008), (5, 4096, 14336),
                                   (8, 2048, 16), (9, 4096, 4096), (16, 4096, 12289),
                                   (16, 2048, 7), (13, 4096, 16400), (4, 4096, 1), (2, 4096, 300),
                                   (11, 2048, 16383), (8, 4096, 11008), (2, 4096, 11008),
                                   (4, 2048, 11008), (6, 4096, 5000), (16, 2048, 16383),
                                   (7, 4096, 16384)])
def test_w8a8_gemv_balanced_rows(dev, hip, m, k, n):
    """The balanced-row GEMV (M <= 16, K = 2048 or 4096, up to 64 rows per
    workgroup on a 256-CU part): 1-4 tiles per workgroup (load windows of 4
    and 8 units, the last tiles' units issued while the first compute), row
    ranges that are not multiples of 16 (the last tile padded with zero rows
    read past the range's buffer descriptor), fewer rows than CUs, rows past
    M, exactly 64 rows per CU, and a shape with more than 64 rows per CU (the
    per-tile kernel) -- int32 and fp32 bit-exact against the oracle, with
    bias + ReLU and with the accumulator alone."""
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=5 * m + n + k, outliers=0.01)
    ye, acce = O.w8a8_linear(aq, sa, wq, sw, bias, True)
    d = [to_dev(a, dev) for a in (aq, sa, wq, sw, bias)]
    y, acc = hip.w8a8_linear(*d, relu=True, want_acc=True)
    assert np.array_equal(host(acc), acce)
    assert_f32_equal(host(y), ye)
    _, acc2 = hip.w8a8_linear(d[0], None, d[2], None, None, want_y=False, want_acc=True)
    assert np.array_equal(host(acc2), acce)


@pytest.mark.parametrize("k,n", [(4096, 512), (4096, 1001), (8192, 1025), (65536, 513),
                                 (69632, 520), (4096, 511), (12288, 11008)])
def test_w8a8_gemv_single_row(dev, hip, k, n):
    """The single-row GEMV (M = 1, K % 4096 == 0, K <= 65536, N >= 512): odd N
    (the last workgroup's second wave stores nothing), several 4 KiB K
    chunks, the largest K it takes, and the shapes just outside it (K =
    69632, N = 511: the other kernels) -- int32 and fp32 bit-exact against
    the oracle with bias + ReLU and with the accumulator alone, and equal to
    the tiled kernel bit for bit. Activations with outliers and the int8
    extremes -128 / 127 in both operands."""
    aq, sa, wq, sw, bias = w8a8_case(1, k, n, seed=k + n, outliers=0.01)
    aq[0, :64] = -128
    aq[0, 64:128] = 127
    wq[:3, :128] = -128
    wq[3:6, :128] = 127
    ye, acce = O.w8a8_linear(aq, sa, wq, sw, bias, True)
    d = [to_dev(a, dev) for a in (aq, sa, wq, sw, bias)]
    y, acc = hip.w8a8_linear(*d, relu=True, want_acc=True)
    assert np.array_equal(host(acc), acce)
    assert_f32_equal(host(y), ye)
    _, acc2 = hip.w8a8_linear(d[0], None, d[2], None, None, want_y=False, want_acc=True)
    assert np.array_equal(host(acc2), acce)
    y3, acc3 = hip.w8a8_linear(*d, relu=True, want_acc=True, algo=hip.ALGO_TILED)
    assert np.array_equal(host(acc3), acce) and np.array_equal(host(y3), host(y))


def test_igemm_single_row_gemv(dev, hip):
    """igemm at M = 1 above the one-launch size (m n k > 2^28): the packed
    operands go through the single-row GEMV with the zero-point column sums
    in its epilogue, against the oracle over the full u8 range."""
    m, k, n = 1, 4096, 70000
    a = (np.arange(m * k) % 251).astype(np.uint8).reshape(m, k)
    b = (np.arange(k * n) % 255).astype(np.uint8).view(np.int8).reshape(k, n)
    import torch
    ws = torch.empty(hip.igemm_workspace_size(m, k, n), dtype=torch.uint8, device=dev)
    got = host(hip.igemm(to_dev(a, dev), to_dev(b, dev), m, k, n, workspace=ws))
    exp, _ = O.igemm(a, b, m, k, n, 8)
    assert np.array_equal(got, exp)


def test_w8a8_prefill_full_size_sampled_rows(dev, hip):
    """BASELINE prefill config (2048 x 4096 x 14336): every output of 24
    sampled rows (covering all 16 row tiles) against the oracle, plus the
    row-sum identity sum_n acc[m,n] = a[m,:] . (sum_n w[n,:]) for all rows."""
    import torch
    c = W.PREFILL
    m, k, n = c["m"], c["k"], c["n"]
    aq, sa, wq, sw, _ = w8a8_case(m, k, n, seed=99)
    y, acc = hip.w8a8_linear(to_dev(aq, dev), to_dev(sa, dev), to_dev(wq, dev), to_dev(sw, dev),
                             want_acc=True)
    rows = np.unique(np.concatenate([np.arange(0, m, 128) + 127, W.rng(1).integers(0, m, 8)]))
    ye, acce = O.w8a8_linear(aq[rows], sa[rows], wq, sw)
    assert np.array_equal(host(acc[torch.as_tensor(rows, device=dev)]), acce)
    assert_f32_equal(host(y[torch.as_tensor(rows, device=dev)]), ye)
    wsum = wq.astype(np.int64).sum(axis=0)
    rowsum = aq.astype(np.int64) @ wsum
    got = host(acc.to(torch.int64).sum(dim=1))
    assert np.array_equal(got, rowsum)


def test_w8a8_mlp_784_256_128_10(dev, hip):
    """int8 MLP 784-256-128-10, batch 32, per-channel
    weights, per-row activations, bias + ReLU between layers, chained on the
    device (quantize -> W8A8 -> quantize ...) against the oracle chain."""
    layers = W.MLP_LAYERS
    x = W.activations(W.MLP_BATCH, layers[0], seed=1)
    params = []
    for i, (fi, fo) in enumerate(zip(layers[:-1], layers[1:])):
        wq, sw = O.quant_rows_i8(W.weights(fo, fi, seed=10 + i))
        b = W.weights(1, fo, seed=20 + i)[0]
        params.append((wq, sw, b))
    h_ref = x
    h = to_dev(x, dev)
    for i, (wq, sw, b) in enumerate(params):
        relu = i < len(params) - 1
        aq, sa = O.quant_rows_i8(h_ref)
        h_ref, _ = O.w8a8_linear(aq, sa, wq, sw, b, relu)
        aq_d, sa_d = hip.quant_rows_i8(h)
        h, _ = hip.w8a8_linear(aq_d, sa_d, to_dev(wq, dev), to_dev(sw, dev), to_dev(b, dev),
                               relu=relu)
    assert_f32_equal(host(h), h_ref)


@pytest.mark.parametrize("m,k,n", [(1, 1, 5), (3, 7, 17), (5, 100, 33), (40, 257, 65),
                                   (32, 787, 256), (130, 300, 129)])
def test_w8a8_any_k_and_unaligned_operands(dev, hip, m, k, n):
    """k % 16 != 0 and operands at odd byte addresses: the reference's igemm
    takes any K (src/int8.rs:288-296), and AUTO routes such calls to the
    byte-assembling tiled kernel. int32 and fp32 bit-exact."""
    import torch
    aq, sa, wq, sw, bias = w8a8_case(m, k, n, seed=3 * m + k)
    for relu, b in ((False, None), (True, bias)):
        y, acc = run_w8a8(dev, hip, aq, sa, wq, sw, b, relu, hip.ALGO_AUTO)
        ye, acce = O.w8a8_linear(aq, sa, wq, sw, b, relu)
        assert np.array_equal(acc, acce)
        assert_f32_equal(y, ye)
    # the same operands one byte past an aligned address (k % 16 == 0 here too)
    for mm, kk, nn in ((m, k, n), (8, 64, 24)):
        aq2, sa2, wq2, sw2, _ = w8a8_case(mm, kk, nn, seed=mm + kk)
        abuf = torch.zeros(mm * kk + 1, dtype=torch.int8, device=dev)
        wbuf = torch.zeros(nn * kk + 1, dtype=torch.int8, device=dev)
        abuf[1:] = to_dev(aq2.reshape(-1), dev)
        wbuf[1:] = to_dev(wq2.reshape(-1), dev)
        y2, acc2 = hip.w8a8_linear(abuf[1:].view(mm, kk), to_dev(sa2, dev), wbuf[1:].view(nn, kk),
                                   to_dev(sw2, dev), want_acc=True)
        ye2, acce2 = O.w8a8_linear(aq2, sa2, wq2, sw2)
        assert np.array_equal(host(acc2), acce2)
        assert_f32_equal(host(y2), ye2)
