"""GPU parity of the QuantizedTensor formats (src/quantize.rs) through the C
ABI against the oracle.

- quantize: data bytes and scales bit-exact, every format, ragged groups
  (odd sizes, a short last group, group 0 = whole tensor, groups above the
  one-wave-per-group limit), zero groups, NaN/Inf/signed zero, half and
  bfloat edge values;
- dequantize: bit-exact on the oracle's codes, including a shortened scales
  array (scales[min(i/group, len-1)]) and the odd-group 4-bit layout;
- QuantizedLinear::forward: f32 sums in the kernel's own order, so the bar is
  the GEMM rounding bound |got - exact| <= gamma_(k+2) * sum |x||W| (+ |b| u)
  around the float64 product of the oracle's dequantized weight (gamma_j =
  j u / (1 - j u), u = 2^-24); the VALU GEMV, the f32-MFMA GEMV and the
  dequantize + f32 GEMM path are each forced on the same inputs.
"""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

ALL = [O.QF_FP16, O.QF_BF16, O.QF_INT8, O.QF_INT4, O.QF_NF4, O.QF_NVFP4, O.QF_GGUF_Q4,
       O.QF_GGUF_Q4K, O.QF_GGUF_Q8]
GEMV_FMTS = [O.QF_INT4, O.QF_INT8, O.QF_GGUF_Q4, O.QF_GGUF_Q8, O.QF_FP16, O.QF_BF16, O.QF_NF4,
             O.QF_NVFP4]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.cpu().numpy()


def weights(n, seed, scale=0.02):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(n) * scale).astype(np.float32)


def special(n, seed):
    """Normal data with zero runs, NaN, +-Inf, signed zeros, huge/tiny values
    and exact code midpoints."""
    x = weights(n, seed, 1.0)
    rng = np.random.default_rng(seed + 1)
    idx = rng.choice(n, size=min(n, 40), replace=False)
    vals = np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 3e38, -3e38, 1e-40, -1e-42, 65504.0,
                     65520.0, 6e-8, 0.5, -0.5, 1.5, 2.5], np.float32)
    x[idx] = vals[np.arange(idx.size) % vals.size]
    if n >= 96:
        x[32:64] = 0.0
    return x


def check_quantize(hip, dev, fmt, x, gs):
    d, s, g = hip.qt_quantize(fmt, to_dev(x, dev), gs)
    de, se, ge = O.qt_quantize(fmt, x, gs)
    assert g == ge
    assert np.array_equal(host(d), de), f"{O.QF_NAMES[fmt]}: codes differ"
    assert np.array_equal(host(s).view(np.uint32), se.view(np.uint32)), "scales differ"
    out = host(hip.qt_dequantize(fmt, d, s, g, x.size))
    exp = O.qt_dequantize(fmt, de, se, ge, x.size)
    assert np.array_equal(out.view(np.uint32), exp.view(np.uint32)), "dequantize differs"


@pytest.mark.parametrize("fmt", ALL, ids=[O.QF_NAMES[f] for f in ALL])
@pytest.mark.parametrize("n,gs", [(4096, 32), (4096, 128), (1000, 33), (999, 7), (77, 0),
                                  (1, 0), (5, 64), (20000, 10000), (30001, 0), (65, 64)])
def test_quantize_dequantize_parity(dev, hip, fmt, n, gs):
    check_quantize(hip, dev, fmt, weights(n, n * 13 + gs), gs)


@pytest.mark.parametrize("fmt", ALL, ids=[O.QF_NAMES[f] for f in ALL])
def test_quantize_special_values(dev, hip, fmt):
    for n, gs in ((4096, 32), (333, 11), (9000, 0)):
        check_quantize(hip, dev, fmt, special(n, n + gs), gs)


def test_half_conversions_every_pattern(dev, hip):
    """FP16/BF16 dequantize of all 65,536 bit patterns, and quantize of their
    f32 values plus random floats of every magnitude."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    for fmt in (O.QF_FP16, O.QF_BF16):
        out = host(hip.qt_dequantize(fmt, to_dev(h.view(np.uint8), dev),
                                     to_dev(np.zeros(1, np.float32), dev), 0, h.size))
        exp = O.qt_dequantize(fmt, h.view(np.uint8), np.zeros(0, np.float32), 0, h.size)
        assert np.array_equal(out.view(np.uint32), exp.view(np.uint32))
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-45, 38, 50000)).astype(np.float32)
    x = np.concatenate([x, h.view(np.float16).astype(np.float32),
                        np.array([0x7F800001, 0xFFFFFFFF, 0x7FC00000], np.uint32).view(np.float32)])
    for fmt in (O.QF_FP16, O.QF_BF16):
        check_quantize(hip, dev, fmt, x, 0)


def test_dequantize_short_scales_and_odd_groups(dev, hip):
    """scales[min(i/group, len-1)] with a caller-shortened scales array, and
    the odd-group INT4 layout read through data[i/2] (src/quantize.rs:377-396);
    groups of 33 over 1001 elements take the one-element kernel, groups of 32
    and 40 over 1024 the eight-element one (power-of-two shift and division)."""
    for n, gs in ((1001, 33), (1024, 32), (1040, 40)):
        x = weights(n, 5 + gs, 1.0)
        for fmt in (O.QF_INT8, O.QF_INT4, O.QF_NF4, O.QF_NVFP4):
            d, s, g = O.qt_quantize(fmt, x, gs)
            for ns in (s.size, 5, 1):
                out = host(hip.qt_dequantize(fmt, to_dev(d, dev), to_dev(s[:ns], dev), g, x.size))
                exp = O.qt_dequantize(fmt, d, s[:ns], g, x.size)
                assert np.array_equal(out.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("fmt,gs", [(O.QF_INT4, 128), (O.QF_INT8, 64), (O.QF_INT4, 32)],
                         ids=["INT4-g128", "INT8-g64", "INT4-g32"])
def test_linear_forward_short_scales(dev, hip, fmt, gs):
    """QuantizedLinear::forward with a caller-shortened scales array (the
    reference reads scales[min(i/group, len-1)]): every fused path that takes
    it -- the VALU GEMV, the f32-MFMA GEMV, AUTO at m = 1 and 8 -- matches the
    dequantized weight within the GEMM bound; the bf16 GEMV, which reads a
    row's scales as a run, refuses it when forced."""
    rng = np.random.default_rng(gs + fmt)
    n, k = 300, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    d, s, g = O.qt_quantize(fmt, w, gs)
    for ns in (s.size // 2 + 3, 1):
        sh = s[:ns]
        wdeq = O.qt_dequantize(fmt, d, sh, g, n * k).reshape(n, k)
        dd, sd = to_dev(d, dev), to_dev(sh, dev)
        for m in (1, 8):
            x = rng.standard_normal((m, k)).astype(np.float32)
            xd = to_dev(x, dev)
            for algo in (None, hip.ALGO_GEMV, hip.ALGO_GEMV_MFMA):
                kw = {} if algo is None else {"algo": algo}
                gemm_check(host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, **kw)), x, wdeq, None)
            with pytest.raises(hip.RnnError):
                hip.qt_linear_forward(fmt, xd, dd, sd, g, n, algo=hip.ALGO_GEMV_BF16)


def test_argument_errors(dev, hip):
    import torch
    x = torch.zeros(64, device=dev)
    with pytest.raises(hip.RnnError):
        hip.qt_quantize(99, x, 32)
    d, s, g = hip.qt_quantize(O.QF_INT4, x, 32)
    with pytest.raises(hip.RnnError):          # data shorter than the tensor needs
        hip.qt_dequantize(O.QF_INT4, d[:10], s, g, 64)
    with pytest.raises(hip.RnnError):          # no scales
        hip.qt_dequantize(O.QF_INT4, d, s[:0], g, 64)
    xr = torch.zeros((2, 48), device=dev)
    d, s, g = hip.qt_quantize(O.QF_INT4, torch.zeros(48 * 8, device=dev), 48)
    with pytest.raises(hip.RnnError):          # forced GEMV: in_f % 32 != 0
        hip.qt_linear_forward(O.QF_INT4, xr, d, s, g, 8, algo=hip.ALGO_GEMV)
    with pytest.raises(hip.RnnError):          # forced GEMV: group 48 is not a multiple of 32
        hip.qt_linear_forward(O.QF_NF4, torch.zeros((1, 64), device=dev), d, s, g, 3,
                              algo=hip.ALGO_GEMV)


# ------------------------------------------------------------------ linear forward
def gemm_check(got, x, wdeq, bias):
    xd, wd = x.astype(np.float64), wdeq.astype(np.float64)
    exact = xd @ wd.T
    scale = np.abs(xd) @ np.abs(wd).T
    if bias is not None:
        exact = exact + bias
        scale = scale + np.abs(bias)
    k = x.shape[1]
    u = 2.0 ** -24
    lim = (k + 2) * u / (1 - (k + 2) * u) * scale + 1e-30
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= lim), f"max err {err.max():.3g}, worst excess {(err - lim).max():.3g}"


def bf16_gemv_fits(fmt, m, k, g):
    """The bf16 MFMA GEMV's conditions: integer codes or bf16 weights, whole
    chunks of 4 pieces for each of 8 waves, groups of whole chunks, or groups
    of 32 (one per MFMA step). Any m: above 16 rows it runs per 16-row
    slice."""
    if fmt not in (O.QF_INT4, O.QF_GGUF_Q4, O.QF_GGUF_Q4K, O.QF_INT8, O.QF_GGUF_Q8, O.QF_BF16):
        return False
    ep = 32 if O.QF_BITS[fmt] == 4 else (16 if O.QF_BITS[fmt] == 8 else 8)
    grouped = fmt != O.QF_BF16
    return (k % (32 * ep) == 0 and
            (not grouped or (g % (4 * ep) == 0 and k % g == 0) or g % k == 0 or g == 32))


@pytest.mark.parametrize("fmt", GEMV_FMTS, ids=[O.QF_NAMES[f] for f in GEMV_FMTS])
@pytest.mark.parametrize("m,k,n,gs", [(1, 4096, 1000, 128), (3, 2048, 257, 32), (4, 64, 9, 64),
                                      (8, 4096, 512, 32), (16, 2080, 130, 32), (2, 6144, 40, 0),
                                      (5, 96, 1, 32), (16, 1024, 33, 32), (11, 3072, 70, 1024),
                                      (17, 1024, 33, 32), (40, 2048, 130, 128)])
def test_linear_forward_gemv_and_gemm(dev, hip, fmt, m, k, n, gs):
    rng = np.random.default_rng(m * 1000 + k + n)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, :7] *= 20.0                                          # outlier channels
    b = rng.standard_normal(n).astype(np.float32)
    g0 = gs if gs else n * k
    if fmt not in (O.QF_FP16, O.QF_BF16) and g0 % 32:
        pytest.skip("group not a multiple of 32")
    d, s, g = O.qt_quantize(fmt, w, gs)
    wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
    dd, sd, xd = to_dev(d, dev), to_dev(s if s.size else np.zeros(1, np.float32), dev), to_dev(x, dev)
    for bias in (None, b):
        bd = None if bias is None else to_dev(bias, dev)
        ep = 32 if O.QF_BITS[fmt] == 4 else (16 if O.QF_BITS[fmt] == 8 else 8)
        algos = [hip.ALGO_GEMV, hip.ALGO_TILED] + ([hip.ALGO_GEMV_MFMA] if k % (16 * ep) == 0 else [])
        if bf16_gemv_fits(fmt, m, k, g):
            algos.append(hip.ALGO_GEMV_BF16)
        for algo in algos:
            y = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, bd, algo=algo))
            gemm_check(y, x, wdeq, bias)
        auto = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, bd))
        gemm_check(auto, x, wdeq, bias)


@pytest.mark.parametrize("fmt,gs", [(O.QF_INT4, 128), (O.QF_INT4, 0), (O.QF_INT8, 64),
                                    (O.QF_INT8, 4096), (O.QF_BF16, 0), (O.QF_INT4, 512),
                                    (O.QF_GGUF_Q8, 32), (O.QF_GGUF_Q4, 32), (O.QF_INT8, 32),
                                    (O.QF_INT4, 32)],
                         ids=["INT4-g128", "INT4-tensor", "INT8-g64", "INT8-rows", "BF16", "INT4-g512",
                              "Q8_0", "Q4_0", "INT8-g32", "INT4-g32"])
@pytest.mark.parametrize("m,k,n", [(5, 4096, 4096), (16, 4096, 5000), (9, 2048, 11008),
                                   (16, 4096, 16000), (12, 1024, 20000), (7, 4096, 30),
                                   (16, 2048, 1),
                                   # three chunks per wave (4-bit codes): weight pairs that
                                   # start mid-line and a last pair with one chunk
                                   (11, 3072, 700),
                                   # long K, few rows: K split 8 ways, one and two chunks per wave
                                   (16, 8192, 300), (16, 16384, 64)])
def test_linear_forward_bf16_gemv(dev, hip, fmt, gs, m, k, n):
    """The bf16 MFMA GEMV (x split into three bf16 parts, codes exact in
    bf16, one scale per group sum -- for groups of 32 one per MFMA step, the
    pieces traded between lane groups --, K split over 1-8 workgroups as the
    plan's estimate picks): 1-12 row tiles per range, one or several chunks
    per wave (x staged through LDS; the weights of two chunks staged as
    whole lines, an odd count of chunks included), row ranges that are not
    multiples of 16, fewer rows than CUs, rows of x past m; with and without
    bias, forced, with the caller's workspace (bit-identical, and the same
    counters reused) and as AUTO picks it, within the GEMM rounding bound; x
    with outlier channels and tiny values."""
    rng = np.random.default_rng(m * 7 + k + n + gs)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, :7] *= 20.0
    x[0, 7:15] = np.float32(3e-30)
    b = rng.standard_normal(n).astype(np.float32)
    if gs == 4096 and k % gs and gs % k:
        gs = k          # "rows": one group per row of W
    d, s, g = O.qt_quantize(fmt, w, gs)
    assert bf16_gemv_fits(fmt, m, k, g)
    wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
    dd, sd, xd = to_dev(d, dev), to_dev(s if s.size else np.zeros(1, np.float32), dev), to_dev(x, dev)
    import torch
    ws = torch.zeros(hip.qt_linear_workspace_size(k, n), dtype=torch.uint8, device=dev)
    for bias in (None, b):
        bd = None if bias is None else to_dev(bias, dev)
        y = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, bd, algo=hip.ALGO_GEMV_BF16))
        gemm_check(y, x, wdeq, bias)
        y2 = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, bd, algo=hip.ALGO_GEMV_BF16,
                                        workspace=ws))
        assert np.array_equal(y2, y)        # same kernels, caller's scratch
    auto = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, to_dev(b, dev)))
    gemm_check(auto, x, wdeq, b)
    # the same workspace for a second x: no partial sum of the first call
    # may survive into the second
    x2 = (rng.standard_normal((m, k)) * 3.0).astype(np.float32)
    y3 = host(hip.qt_linear_forward(fmt, to_dev(x2, dev), dd, sd, g, n, algo=hip.ALGO_GEMV_BF16,
                                    workspace=ws))
    gemm_check(y3, x2, wdeq, None)


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_linear_forward_nonfinite_x(dev, hip, m):
    """Inf, -Inf and NaN in x (a canonical NaN and one whose payload sits
    only in the low 16 bits, which the bf16 split must not turn into an
    infinity): every fused path gives the reference's non-finite pattern --
    inf * w is +-inf, inf * 0 and inf - inf are NaN, whatever the summation
    order -- and its finite outputs stay within the GEMM bound."""
    rng = np.random.default_rng(m + 40)
    n, k = 48, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    w[5, :] = 0.0                                            # inf * 0 -> NaN in column 5
    d, s, g = O.qt_quantize(O.QF_INT4, w, 128)
    wdeq = O.qt_dequantize(O.QF_INT4, d, s, g, n * k).reshape(n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    low_nan = np.array([0x7F800001], dtype=np.uint32).view(np.float32)[0]
    x[0, 10] = np.inf
    if m > 1:
        x[1, 20], x[1, 30] = np.inf, -np.inf                 # +inf - inf -> NaN
    if m > 2:
        x[2, 40] = np.nan
    if m > 3:
        x[3, 50] = low_nan
    with np.errstate(invalid="ignore", over="ignore"):
        ref = O.qt_linear_forward(O.QF_INT4, x, d, s, g, n, None)
    fin = np.isfinite(x).all(axis=1)
    algos = [hip.ALGO_GEMV, hip.ALGO_GEMV_MFMA] + ([hip.ALGO_GEMV_BF16] if m >= 3 else [])
    for algo in algos:
        y = host(hip.qt_linear_forward(O.QF_INT4, to_dev(x, dev), to_dev(d, dev), to_dev(s, dev),
                                       g, n, algo=algo))
        assert np.array_equal(np.isnan(y), np.isnan(ref)), algo
        assert np.array_equal(np.isposinf(y), np.isposinf(ref)), algo
        assert np.array_equal(np.isneginf(y), np.isneginf(ref)), algo
        if fin.any():
            gemm_check(y[fin], x[fin], wdeq, None)


@pytest.mark.parametrize("fmt", [O.QF_GGUF_Q4, O.QF_GGUF_Q8], ids=["Q4_0", "Q8_0"])
@pytest.mark.parametrize("m", [3, 4])
def test_linear_forward_groups_of_32_few_rows(dev, hip, fmt, m):
    """GGUF blocks of 32 at m = 3, 4 and N = 11008 (three row tiles per CU):
    AUTO takes the bf16 GEMV for 4- and 8-bit codes (one MFMA step per group,
    the pieces read from the staged weight lines in the step's order) -- the
    same bits as the bf16 GEMV forced --, and the VALU GEMV forced; all
    within the GEMM bound."""
    rng = np.random.default_rng(90 + m + fmt)
    n, k = 11008, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[:, :5] *= 30.0
    d, s, g = O.qt_quantize(fmt, w, 32)
    assert g == 32 and bf16_gemv_fits(fmt, m, k, g)
    wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
    dd, sd, xd = to_dev(d, dev), to_dev(s, dev), to_dev(x, dev)
    auto = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n))
    gemm_check(auto, x, wdeq, None)
    bf16 = host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, algo=hip.ALGO_GEMV_BF16))
    assert np.array_equal(auto, bf16)
    gemm_check(host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, algo=hip.ALGO_GEMV)), x, wdeq, None)


def test_linear_forward_groups_of_32_unaligned_scales(dev, hip):
    """GGUF Q8_0 at m = 8 with its scales 4 bytes past a 16-byte boundary: the
    bf16 GEMV reads a chunk's scales in one vector load, so AUTO takes
    another fused path (within the GEMM bound) and the forced bf16 GEMV
    refuses the call."""
    import torch
    rng = np.random.default_rng(77)
    n, k, m = 1000, 4096, 8
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    d, s, g = O.qt_quantize(O.QF_GGUF_Q8, w, 32)
    wdeq = O.qt_dequantize(O.QF_GGUF_Q8, d, s, g, n * k).reshape(n, k)
    buf = torch.zeros(s.size + 1, dtype=torch.float32, device=dev)
    buf[1:] = torch.from_numpy(s).to(dev)
    sd = buf[1:]
    assert sd.data_ptr() % 16 == 4
    dd, xd = to_dev(d, dev), to_dev(x, dev)
    gemm_check(host(hip.qt_linear_forward(O.QF_GGUF_Q8, xd, dd, sd, g, n)), x, wdeq, None)
    with pytest.raises(hip.RnnError):
        hip.qt_linear_forward(O.QF_GGUF_Q8, xd, dd, sd, g, n, algo=hip.ALGO_GEMV_BF16)


@pytest.mark.parametrize("fmt,gs", [(O.QF_INT4, 128), (O.QF_GGUF_Q8, 32), (O.QF_NF4, 64),
                                    (O.QF_FP16, 0)], ids=["INT4-g128", "GGUF-Q8_0", "NF4-g64", "FP16"])
def test_linear_forward_row_slices(dev, hip, fmt, gs):
    """Above 16 rows the GEMVs run on 16-row slices of x and y: AUTO at m = 40
    is bit-identical to AUTO on rows 0-15, 16-31 and 32-39 called one by one
    (the slice offsets), and every route -- AUTO within and beyond its slice
    limit (m = 600: dequantize + f32 GEMM for every format) and each
    forced GEMV -- is within the f32 GEMM bound of the dequantized weight."""
    import torch
    rng = np.random.default_rng(40 + fmt)
    n, k = 200, 2048
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    d, s, g = O.qt_quantize(fmt, w, gs)
    wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
    dd, sd = to_dev(d, dev), to_dev(s if s.size else np.zeros(1, np.float32), dev)
    x = rng.standard_normal((600, k)).astype(np.float32)
    xd = to_dev(x, dev)
    b = rng.standard_normal(n).astype(np.float32)
    bd = to_dev(b, dev)
    y40 = host(hip.qt_linear_forward(fmt, xd[:40], dd, sd, g, n, bd))
    parts = [host(hip.qt_linear_forward(fmt, xd[a:e], dd, sd, g, n, bd))
             for a, e in ((0, 16), (16, 32), (32, 40))]
    np.testing.assert_array_equal(y40, np.concatenate(parts))
    gemm_check(y40, x[:40], wdeq, b)
    gemm_check(host(hip.qt_linear_forward(fmt, xd, dd, sd, g, n, bd)), x, wdeq, b)
    algos = [hip.ALGO_GEMV, hip.ALGO_GEMV_MFMA, hip.ALGO_TILED]
    if bf16_gemv_fits(fmt, 40, k, g):
        algos.append(hip.ALGO_GEMV_BF16)
    for algo in algos:
        y = torch.full((40, n), float("nan"), device=dev)
        hip.qt_linear_forward(fmt, xd[:40], dd, sd, g, n, bd, algo=algo, y=y)
        gemm_check(host(y), x[:40], wdeq, b)


def test_linear_forward_bf16_gemv_rejects(dev, hip):
    """Forced bf16 GEMV outside its conditions: NF4 codes, GGUF Q4_0 and
    INT4 with in_f = 512 (4-bit chunks need in_f % 1024 == 0; at m = 17 the
    first 16-row slice refuses); and a workspace one 16-byte step too small
    -- an RnnError, no launch."""
    rng = np.random.default_rng(3)
    n, k = 64, 512
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    for fmt, gs, m in ((O.QF_NF4, 128, 8), (O.QF_GGUF_Q4, 32, 8), (O.QF_INT4, 128, 17)):
        d, s, g = O.qt_quantize(fmt, w, gs)
        x = to_dev(rng.standard_normal((m, k)).astype(np.float32), dev)
        with pytest.raises(hip.RnnError) as e:
            hip.qt_linear_forward(fmt, x, to_dev(d, dev), to_dev(s, dev), g, n,
                                  algo=hip.ALGO_GEMV_BF16)
        assert e.value.status == hip.RNN_ERR_INVALID_ARG or e.value.status == hip.RNN_ERR_UNSUPPORTED
    # a workspace below rnn_qt_linear_workspace_size
    import torch
    d, s, g = O.qt_quantize(O.QF_INT4, w, 128)
    small = torch.empty(hip.qt_linear_workspace_size(k, n) - 16, dtype=torch.uint8, device=dev)
    with pytest.raises(hip.RnnError) as e:
        hip.qt_linear_forward(O.QF_INT4, to_dev(rng.standard_normal((8, k)).astype(np.float32), dev),
                              to_dev(d, dev), to_dev(s, dev), g, n, workspace=small)
    assert e.value.status == hip.RNN_ERR_INVALID_ARG


@pytest.mark.parametrize("fmt", [O.QF_NF4, O.QF_NVFP4, O.QF_INT4],
                         ids=["NF4", "NVFP4", "INT4-odd-group"])
def test_linear_forward_dequant_path(dev, hip, fmt):
    """Shapes outside the fused GEMV (in_f = 200 is not a multiple of 32, a
    group of 33) take dequantize + f32 GEMM, for m = 1 and 40."""
    rng = np.random.default_rng(fmt)
    n, k = 70, 200
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    gs = 33 if fmt == O.QF_INT4 else 64
    d, s, g = O.qt_quantize(fmt, w, gs)
    wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
    b = rng.standard_normal(n).astype(np.float32)
    for m in (1, 40):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = host(hip.qt_linear_forward(fmt, to_dev(x, dev), to_dev(d, dev), to_dev(s, dev), g, n,
                                       to_dev(b, dev)))
        gemm_check(y, x, wdeq, b)
        assert np.abs(y - O.qt_linear_forward(fmt, x, d, s, g, n, b)).max() < 1e-3


def test_linear_forward_decode_config_sampled(dev, hip):
    """The bench workload: INT4 group 128 and GGUF Q4_0/Q8_0 weights
    [11008, 4096], x [1, 4096] and [4, 4096]; every output checked."""
    rng = np.random.default_rng(77)
    n, k = 11008, 4096
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    for fmt, gs in ((O.QF_INT4, 128), (O.QF_GGUF_Q4, 32), (O.QF_GGUF_Q8, 32)):
        d, s, g = O.qt_quantize(fmt, w, gs)
        dq, sq, _ = hip.qt_quantize(fmt, to_dev(w, dev), gs)
        assert np.array_equal(host(dq), d) and np.array_equal(host(sq), s)
        wdeq = O.qt_dequantize(fmt, d, s, g, n * k).reshape(n, k)
        for m in (1, 4, 16):
            x = rng.standard_normal((m, k)).astype(np.float32)
            y = host(hip.qt_linear_forward(fmt, to_dev(x, dev), dq, sq, g, n))
            gemm_check(y, x, wdeq, None)


def test_quantized_layers(dev, hip):
    """QuantizedTensor / QuantizedLinear / QuantizedModel mirrors
    (src/quantize.rs:214-816): sizes, ratios, the from_model pairing and a
    forward through each layer."""
    import torch
    import layers as L
    rng = np.random.default_rng(3)
    params = [rng.standard_normal((128, 64)).astype(np.float32) * 0.05,
              rng.standard_normal(128).astype(np.float32),
              rng.standard_normal((64, 128)).astype(np.float32) * 0.05,
              rng.standard_normal(64).astype(np.float32)]
    tp = [to_dev(p, dev) for p in params]
    qm = L.QuantizedModel.from_model(tp, O.QF_INT4, 32)
    assert len(qm.layers()) == 2
    nbytes = sum(O.qt_layout(O.QF_INT4, p.size, 32)[0] + 4 * O.qt_layout(O.QF_INT4, p.size, 32)[1]
                 for p in params[::2])
    assert qm.mem_bytes() == nbytes + 4 * (128 + 64)
    assert qm.compression_ratio() > 4.0                  # quantized_model_compression
    x = rng.standard_normal((2, 64)).astype(np.float32)
    h = x
    for i, layer in enumerate(qm.layers()):
        y = host(layer.forward(to_dev(h, dev)))
        d, s, g = O.qt_quantize(O.QF_INT4, params[2 * i], 32)
        wdeq = O.qt_dequantize(O.QF_INT4, d, s, g, params[2 * i].size).reshape(params[2 * i].shape)
        gemm_check(y, h, wdeq, params[2 * i + 1])
        h = y
    qt = L.QuantizedTensor.quantize(tp[0], O.QF_NF4, 64)
    assert qt.dequantize().shape == (128, 64)
    assert abs(qt.compression_ratio() - 128 * 64 * 4 / (128 * 64 / 2 + 4 * 128)) < 1e-9
    assert qt.quantization_error(tp[0]) < 0.05 * 0.2
    ql = L.QuantizedLinear.from_linear(tp[2], None, O.QF_INT8, 0)   # quantized_linear_forward
    assert tuple(ql.forward(torch.zeros((2, 128), device=dev)).shape) == (2, 64)
