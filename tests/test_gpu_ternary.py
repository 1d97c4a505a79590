"""GPU parity: ternary packing, quantization, dequantization, the reference
f32 TernaryLinear::forward and the int8-MFMA ternary GEMM, against the oracle
(bit-exact codes, scales, int32 accumulators and fp32 outputs)."""
import numpy as np
import pytest

import oracle as O
import workloads as W
from test_gpu_int8 import assert_f32_equal, host, to_dev

pytestmark = pytest.mark.gpu


def rand_ternary(n, k, seed, with_code3=False):
    g = W.rng(seed)
    t = g.integers(-1, 2, (n, k)).astype(np.int8)
    p = O.pack_ternary(t)
    if with_code3:  # sprinkle unused code 11 (decodes to 0, src/ternary.rs:71)
        sel = g.random(p.size) < 0.2
        p = np.where(sel, p | np.uint32(0x3 << 6), p).astype(np.uint32)
        t = O.unpack_ternary(p, n * k).reshape(n, k)
    return t, p


@pytest.mark.parametrize("count", [16, 1000, 1, 17, 4096 * 64])
def test_pack_unpack_parity(dev, hip, count):
    t = W.rng(count).integers(-1, 2, count).astype(np.int8)
    t[::7] = 5  # any v > 0 packs to 01 (src/ternary.rs:54)
    p = host(hip.ternary_pack(to_dev(t, dev))).view(np.uint32)
    assert np.array_equal(p, O.pack_ternary(t))
    u = host(hip.ternary_unpack(to_dev(p.view(np.int32), dev), count))
    assert np.array_equal(u, O.unpack_ternary(p, count))


def test_pack_known_word(dev, hip):
    v = np.array([1, -1, 0, 1, -1, 0, 1, 1, -1, -1, 0, 0, 1, -1, 1, 0], np.int8)
    assert host(hip.ternary_pack(to_dev(v, dev))).view(np.uint32).tolist() == [0x190A5249]


@pytest.mark.parametrize("rows,cols", [(2, 4), (64, 128), (37, 19), (512, 4096)])
def test_quantize_rows_parity(dev, hip, rows, cols):
    w = W.weights(rows, cols, seed=rows + cols, std=1.0)
    w[0, : min(cols, 2)] = 0.0
    p, s = hip.ternary_quantize(to_dev(w, dev), hip.TERNARY_ROWS)
    t, so = O.ternary_quantize_rows(w)
    assert np.array_equal(host(s), so)
    assert np.array_equal(host(p).view(np.uint32), O.pack_ternary(t))


@pytest.mark.parametrize("rows,cols", [(64, 128), (37, 19), (4096, 4096)])
def test_quantize_absmean_parity(dev, hip, rows, cols):
    w = W.ternary_latent(rows, cols, seed=rows)
    p, s = hip.ternary_quantize(to_dev(w, dev), hip.TERNARY_ABSMEAN)
    t, g = O.ternary_quantize_absmean(w)
    assert np.all(host(s) == g)
    assert np.array_equal(host(p).view(np.uint32), O.pack_ternary(t))


def test_dequantize_parity(dev, hip):
    n, k = 40, 33
    t, p = rand_ternary(n, k, seed=3, with_code3=True)
    sc = W.rng(4).random(n).astype(np.float32)
    got = host(hip.ternary_dequantize(to_dev(p.view(np.int32), dev), n * k, to_dev(sc, dev), k))
    assert np.array_equal(got, O.ternary_dequantize(p, n * k, sc, k))


@pytest.mark.parametrize("batch,in_f,out_f", [(2, 8, 4), (1, 4, 2), (16, 333, 70), (64, 4096, 512)])
def test_ternary_linear_forward_parity(dev, hip, batch, in_f, out_f):
    """Reference f32 shift-and-add (src/ternary.rs:239-279), sequential in k."""
    t, p = rand_ternary(out_f, in_f, seed=in_f, with_code3=True)
    x = W.activations(batch, in_f, seed=batch)
    sc = W.rng(5).random(out_f).astype(np.float32)
    bias = W.rng(6).standard_normal(out_f).astype(np.float32)
    for b in (None, bias):
        got = host(hip.ternary_linear_forward(to_dev(x, dev), to_dev(p.view(np.int32), dev),
                                              to_dev(sc, dev), out_f,
                                              None if b is None else to_dev(b, dev)))
        assert_f32_equal(got, O.ternary_linear_f32(x, p, sc, out_f, b))


@pytest.mark.parametrize("m,k,n", [(1, 64, 16), (37, 48, 29), (128, 256, 128), (200, 4096, 300)])
def test_ternary_gemm_parity(dev, hip, m, k, n):
    t, p = rand_ternary(n, k, seed=m + n, with_code3=True)
    aq = W.rng(m).integers(-128, 128, (m, k)).astype(np.int8)
    sa = W.rng(m + 1).random(m).astype(np.float32)
    sw = np.full(n, np.float32(0.7979), np.float32)
    bias = W.rng(2).standard_normal(n).astype(np.float32)
    for relu, b in ((False, None), (True, bias)):
        y, acc = hip.ternary_gemm(to_dev(aq, dev), to_dev(sa, dev), to_dev(p.view(np.int32), dev),
                                  to_dev(sw, dev), n, None if b is None else to_dev(b, dev),
                                  relu=relu, want_acc=True)
        ye, acce = O.ternary_gemm_i8(aq, sa, p, sw, n, b, relu)
        assert np.array_equal(host(acc), acce)
        assert_f32_equal(host(y), ye)


@pytest.mark.parametrize("m,k,n", [(128, 128, 64), (200, 4096, 300), (17, 256, 4), (512, 1024, 452),
                                   (300, 384, 1000)])
@pytest.mark.parametrize("algo", ["tiled", "dma"])
def test_ternary_gemm_forced_kernels(dev, hip, m, k, n, algo):
    """Both ternary kernels, forced: the register-staged 128x128 tiles and the
    LDS-DMA 128x64 tiles whose 2-bit words are decoded through an LDS table,
    with ragged M/N edges; int32 and fp32 bit-exact."""
    t, p = rand_ternary(n, k, seed=3 * m + n, with_code3=True)
    aq = W.rng(m + 5).integers(-128, 128, (m, k)).astype(np.int8)
    sa = W.rng(m + 6).random(m).astype(np.float32)
    sw = W.rng(n).random(n).astype(np.float32)
    bias = W.rng(3).standard_normal(n).astype(np.float32)
    a = hip.ALGO_TILED if algo == "tiled" else hip.ALGO_TILED_DMA
    y, acc = hip.ternary_gemm(to_dev(aq, dev), to_dev(sa, dev), to_dev(p.view(np.int32), dev),
                              to_dev(sw, dev), n, to_dev(bias, dev), relu=True, want_acc=True,
                              algo=a)
    ye, acce = O.ternary_gemm_i8(aq, sa, p, sw, n, bias, True)
    assert np.array_equal(host(acc), acce)
    assert_f32_equal(host(y), ye)


def test_ternary_gemm_full_config_sampled(dev, hip):
    """BASELINE ternary config (512 x 4096 x 4096, absmean weights, per-row int8
    activations): 32 sampled rows against the oracle, all rows via the
    row-sum identity."""
    import torch
    c = W.TERNARY
    m, k, n = c["m"], c["k"], c["n"]
    wl = W.ternary_latent(n, k, seed=7)
    t, g = O.ternary_quantize_absmean(wl)
    p = O.pack_ternary(t)
    x = W.activations(m, k, seed=8)
    aq, sa = O.quant_rows_i8(x)
    sw = np.full(n, g, np.float32)
    rows = np.unique(np.concatenate([np.arange(0, m, 16) + 15, [0, 1]]))
    ye, acce = O.ternary_gemm_i8(aq[rows], sa[rows], p, sw, n)
    ridx = torch.as_tensor(rows, device=dev)
    rowsum = aq.astype(np.int64) @ t.astype(np.int64).sum(axis=0)
    pd = to_dev(p.view(np.int32), dev)
    # the reference code layout, then the MFMA layout of rnn_ternary_prepack
    for codes, mfma in ((pd, False), (hip.ternary_prepack(pd, n, k), True)):
        y, acc = hip.ternary_gemm(to_dev(aq, dev), to_dev(sa, dev), codes, to_dev(sw, dev), n,
                                  want_acc=True, mfma_layout=mfma)
        assert np.array_equal(host(acc[ridx]), acce)
        assert_f32_equal(host(y[ridx]), ye)
        assert np.array_equal(host(acc.to(torch.int64).sum(dim=1)), rowsum)


@pytest.mark.parametrize("m,k,n", [(1, 1, 3), (5, 7, 9), (37, 50, 29), (64, 300, 70),
                                   (200, 1001, 33)])
def test_ternary_gemm_any_k(dev, hip, m, k, n):
    """k % 16 != 0: rows of the flat packed codes start mid-word
    (src/ternary.rs:46-60), and AUTO takes the kernel that gathers each row's
    codes from arbitrary bit offsets. int32 and fp32 bit-exact, code 11
    included; also with the activations one byte past an aligned address."""
    import torch
    t, p = rand_ternary(n, k, seed=m + k, with_code3=True)
    aq = W.rng(m + k).integers(-128, 128, (m, k)).astype(np.int8)
    sa = W.rng(m + 1).random(m).astype(np.float32)
    sw = np.full(n, np.float32(0.7979), np.float32)
    bias = W.rng(3).standard_normal(n).astype(np.float32)
    abuf = torch.zeros(m * k + 1, dtype=torch.int8, device=dev)
    abuf[1:] = to_dev(aq.reshape(-1), dev)
    for relu, b in ((False, None), (True, bias)):
        ye, acce = O.ternary_gemm_i8(aq, sa, p, sw, n, b, relu)
        for a_dev in (to_dev(aq, dev), abuf[1:].view(m, k)):
            y, acc = hip.ternary_gemm(a_dev, to_dev(sa, dev), to_dev(p.view(np.int32), dev),
                                      to_dev(sw, dev), n, None if b is None else to_dev(b, dev),
                                      relu=relu, want_acc=True)
            assert np.array_equal(host(acc), acce)
            assert_f32_equal(host(y), ye)


def mfma_layout_np(p):
    """The MFMA code layout, restated independently: code t of each word (bits
    2t) moves to bits 8*(t % 4) + 2*(t // 4)."""
    p = p.astype(np.uint64)
    out = np.zeros_like(p)
    for t in range(16):
        out |= ((p >> np.uint64(2 * t)) & np.uint64(3)) << np.uint64(8 * (t % 4) + 2 * (t // 4))
    return out.astype(np.uint32)


def test_ternary_prepack_layout(dev, hip):
    g = W.rng(77)
    p = g.integers(0, 2**32, 4096, dtype=np.uint64).astype(np.uint32)   # codes 11 included
    got = host(hip.ternary_prepack(to_dev(p.view(np.int32), dev), 64, 1024)).view(np.uint32)
    np.testing.assert_array_equal(got, mfma_layout_np(p))
    with pytest.raises(hip.RnnError):
        hip.ternary_prepack(to_dev(p.view(np.int32), dev), 64, 1000)        # cols % 16 != 0


@pytest.mark.parametrize("m,k,n", [(1, 256, 16), (64, 512, 128), (512, 4096, 512), (37, 48, 29),
                                   (200, 1024, 300), (17, 256, 4), (130, 512, 200),
                                   (96, 1536, 260), (33, 2048, 132), (64, 768, 128)])
def test_ternary_gemm_mfma_layout(dev, hip, m, k, n):
    """The GEMM on prepacked codes (RNN_FLAG_TERNARY_MFMA_LAYOUT) against the
    oracle on the reference layout: the LDS-DMA kernel (k % 256 == 0; one to
    four 128-K stages per K group, ragged M and N edges) and the tiled kernel
    (other k, unaligned activations), int32 and fp32 bit-exact."""
    import torch
    t, p = rand_ternary(n, k, seed=3 * m + n, with_code3=True)
    pm = hip.ternary_prepack(to_dev(p.view(np.int32), dev), n, k)
    aq = W.rng(m + k).integers(-128, 128, (m, k)).astype(np.int8)
    sa = W.rng(m + 2).random(m).astype(np.float32)
    sw = np.full(n, np.float32(0.7979), np.float32)
    bias = W.rng(4).standard_normal(n).astype(np.float32)
    abuf = torch.zeros(m * k + 1, dtype=torch.int8, device=dev)
    abuf[1:] = to_dev(aq.reshape(-1), dev)
    for relu, b in ((False, None), (True, bias)):
        ye, acce = O.ternary_gemm_i8(aq, sa, p, sw, n, b, relu)
        for a_dev in (to_dev(aq, dev), abuf[1:].view(m, k)):
            y, acc = hip.ternary_gemm(a_dev, to_dev(sa, dev), pm, to_dev(sw, dev), n,
                                      None if b is None else to_dev(b, dev), relu=relu,
                                      want_acc=True, mfma_layout=True)
            assert np.array_equal(host(acc), acce)
            assert_f32_equal(host(y), ye)
