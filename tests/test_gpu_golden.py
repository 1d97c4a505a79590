"""GPU parity against the committed golden vectors (tests/golden/golden_small.npz)
through the C ABI, with no oracle in the loop: integer outputs and codes bit-exact,
fp32 outputs within the 1e-5 relative contract (assert_f32_equal demands bit
equality, which is stricter)."""
import os

import numpy as np
import pytest

from test_gpu_int8 import assert_f32_equal, host, to_dev

pytestmark = pytest.mark.gpu

NPZ = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_small.npz")


@pytest.fixture(scope="module")
def G():
    with np.load(NPZ, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("case", ["igemm_kat", "igemm_lcg"])
def test_golden_igemm(dev, hip, G, case):
    a, b = G[f"{case}.a"], G[f"{case}.b"]
    m, k = a.shape
    n = b.shape[1]
    c = hip.igemm(to_dev(a, dev), to_dev(b, dev), m, k, n)
    assert np.array_equal(host(c), G[f"{case}.c"])


def test_golden_quant_rows_and_dequant(dev, hip, G):
    q, s = hip.quant_rows_i8(to_dev(G["quant_rows.x"], dev))
    assert np.array_equal(host(q), G["quant_rows.q"])
    assert np.array_equal(host(s), G["quant_rows.scale"])
    w = hip.int8_dequantize(q, s)
    assert_f32_equal(host(w), G["int8_dequant.w"])


def test_golden_int8_linear(dev, hip, G):
    wq, ws = to_dev(G["int8_lin.wq"], dev), to_dev(G["int8_lin.ws"], dev)
    x, b = to_dev(G["int8_lin.x"], dev), to_dev(G["int8_lin.bias"], dev)
    assert_f32_equal(host(hip.int8_matmul_f32(wq, ws, x)), G["int8_lin.matmul_y"])
    assert_f32_equal(host(hip.int8_linear_forward(x, wq, ws, b)), G["int8_lin.forward_y"])


@pytest.mark.parametrize("algo", ["AUTO", "TILED", "GEMV", "TILED_DMA"])
def test_golden_w8a8(dev, hip, G, algo):
    args = [to_dev(G[f"w8a8.{n}"], dev) for n in ("aq", "sa", "wq", "sw")]
    a = getattr(hip, f"ALGO_{algo}")
    y, acc = hip.w8a8_linear(*args, None, False, algo=a, want_acc=True)
    assert np.array_equal(host(acc), G["w8a8.acc"])
    assert_f32_equal(host(y), G["w8a8.y"])
    y, _ = hip.w8a8_linear(*args, to_dev(G["w8a8.bias"], dev), True, algo=a)
    assert_f32_equal(host(y), G["w8a8.y_bias_relu"])


@pytest.mark.parametrize("case", ["ternary_pack_kat", "ternary_pack_large"])
def test_golden_ternary_pack(dev, hip, G, case):
    t = G[f"{case}.t"]
    p = hip.ternary_pack(to_dev(t, dev))
    assert np.array_equal(host(p).view(np.uint32), G[f"{case}.packed"])
    assert np.array_equal(host(hip.ternary_unpack(p, t.size)), t)


def test_golden_ternary_quantize(dev, hip, G):
    p, s = hip.ternary_quantize(to_dev(G["ternary_rows.w"], dev), hip.TERNARY_ROWS)
    assert np.array_equal(host(p).view(np.uint32), G["ternary_rows.packed"])
    assert np.array_equal(host(s), G["ternary_rows.scale"])
    w = hip.ternary_dequantize(p, G["ternary_rows.w"].size, s, G["ternary_rows.w"].shape[1])
    assert_f32_equal(host(w), G["ternary_dequant.w"])
    p, s = hip.ternary_quantize(to_dev(G["ternary_absmean.w"], dev), hip.TERNARY_ABSMEAN)
    assert np.array_equal(host(p).view(np.uint32), G["ternary_absmean.packed"])
    assert np.all(host(s) == G["ternary_absmean.gamma"][0])


def test_golden_ternary_linear(dev, hip, G):
    p = to_dev(G["ternary_rows.packed"].view(np.int32), dev)
    y = hip.ternary_linear_forward(to_dev(G["ternary_lin.x"], dev), p,
                                   to_dev(G["ternary_rows.scale"], dev), 6,
                                   to_dev(G["ternary_lin.bias"], dev))
    assert_f32_equal(host(y), G["ternary_lin.y"])


@pytest.mark.parametrize("algo", ["AUTO", "TILED", "TILED_DMA"])
def test_golden_ternary_gemm(dev, hip, G, algo):
    aq, sa = to_dev(G["ternary_gemm.aq"], dev), to_dev(G["ternary_gemm.sa"], dev)
    p = to_dev(G["ternary_absmean.packed"].view(np.int32), dev)
    n = 24
    sw = to_dev(np.full(n, G["ternary_absmean.gamma"][0], np.float32), dev)
    a = getattr(hip, f"ALGO_{algo}")
    y, acc = hip.ternary_gemm(aq, sa, p, sw, n, None, False, want_acc=True, algo=a)
    assert np.array_equal(host(acc), G["ternary_gemm.acc"])
    assert_f32_equal(host(y), G["ternary_gemm.y"])
    y, _ = hip.ternary_gemm(aq, sa, p, sw, n, to_dev(G["ternary_gemm.bias"], dev), True, algo=a)
    assert_f32_equal(host(y), G["ternary_gemm.y_bias_relu"])


def test_golden_rotation_matrices(dev, hip, G):
    m = hip.rotation_matrices(to_dev(G["rotor_mats.rotors"], dev))
    assert_f32_equal(host(m), G["rotor_mats.m"])


@pytest.mark.parametrize("case", ["rq_ref.b4", "rq_d128.b3", "rq_d128.b4", "rq_d128.b8",
                                  "rq_d10.b3", "rq_d10.b4", "rq_d10.b8"])
def test_golden_rotorquant(dev, hip, G, case):
    base, b = case.split(".")
    bits = int(b[1:])
    pre = base if base == "rq_ref" else case
    x, r = to_dev(G[f"{base}.x"], dev), to_dev(G[f"{base}.rotors"], dev)
    y, codes, scales = hip.rotorquant_quantize(x, r, bits, want_codes=True)
    assert np.array_equal(host(codes), G[f"{pre}.codes"])
    assert np.array_equal(host(scales), G[f"{pre}.scales"])
    assert_f32_equal(host(y), G[f"{pre}.y"])
    if base != "rq_ref":
        yd = hip.rotorquant_dequantize(codes, scales, x.shape[-1], r)
        assert_f32_equal(host(yd), G[f"{pre}.deq"])


QT_TAGS = ["int8", "nvfp4", "fp16", "rand", "odd"]
QT_NAMES = ["FP16", "BF16", "INT8", "INT4", "NF4", "NVFP4", "GGUF_Q4", "GGUF_Q4K", "GGUF_Q8"]


@pytest.mark.parametrize("tag", QT_TAGS)
def test_golden_quantized_tensor(dev, hip, G, tag):
    """QuantizedTensor::quantize / dequantize (src/quantize.rs:231-269), every
    format: bytes, scales, stored group and values bit-exact."""
    x, gs = G[f"qt_{tag}.x"], int(G[f"qt_{tag}.gs"][0])
    for f, name in enumerate(QT_NAMES):
        key = f"qt_{tag}.{name}"
        d, s, grp = hip.qt_quantize(f, to_dev(x, dev), gs)
        assert grp == int(G[f"{key}.group"][0]), name
        assert np.array_equal(host(d), G[f"{key}.data"]), name
        assert np.array_equal(host(s).view(np.uint32), G[f"{key}.scales"].view(np.uint32)), name
        sd = s if s.numel() else to_dev(np.zeros(1, np.float32), dev)
        out = host(hip.qt_dequantize(f, d, sd, grp, x.size))
        assert np.array_equal(out.view(np.uint32), G[f"{key}.deq"].view(np.uint32)), name


def test_golden_quantized_linear(dev, hip, G):
    """QuantizedLinear::forward (src/quantize.rs:744-754): both GPU paths
    within twice the f32 GEMM bound of the stored oracle output."""
    x, k = G["qt_linear.x"], G["qt_linear.x"].shape[1]
    u = 2.0 ** -24
    tol = 2 * (k + 2) * u / (1 - (k + 2) * u) * G["qt_linear.absdot"] + 1e-30
    for algo in (hip.ALGO_GEMV, hip.ALGO_TILED):
        y = hip.qt_linear_forward(3, to_dev(x, dev), to_dev(G["qt_linear.data"], dev),
                                  to_dev(G["qt_linear.scales"], dev), int(G["qt_linear.group"][0]),
                                  40, to_dev(G["qt_linear.bias"], dev), algo=algo)
        assert np.all(np.abs(host(y).astype(np.float64) - G["qt_linear.y"]) <= tol)


def test_golden_kv_attention(dev, hip, G):
    """Attention over the RotorQuant KV cache (src/tensor.rs:618-672 over the
    4-bit reconstructions) within the stored tolerance of the oracle's output."""
    pages = []
    for kv, kind in (("k", hip.RQ_PAGE_K), ("v", hip.RQ_PAGE_V)):
        pages.append(hip.rotorquant_kv_pack(to_dev(G[f"kv_attn.{kv}_codes"], dev),
                                            to_dev(G[f"kv_attn.{kv}_scales"], dev), 2, 70, 12, 4,
                                            kind))
    out = hip.rotorquant_kv_attention(to_dev(G["kv_attn.q"], dev), pages[0], pages[1],
                                      to_dev(G["kv_attn.k_rotors"], dev),
                                      to_dev(G["kv_attn.v_rotors"], dev), 70, 0.25)
    assert np.all(np.abs(host(out).astype(np.float64) - G["kv_attn.out"]) <= G["kv_attn.tol"])
