"""GPU parity of the layer mirrors (`layers.py`): Int8Weights / Int8Linear
(src/int8.rs:11-172), TernaryTensor / TernaryLinear / TernaryModel
(src/ternary.rs:81-362) and the device-resident Int8Model chain, against the
oracle on the same inputs (fp32 outputs bit for bit)."""
import numpy as np
import pytest

import layers as L
import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def host(t):
    return t.cpu().numpy()


def mlp_params(seed0=10):
    """Module::parameters() of the 784-256-128-10 MLP: weight, bias per layer."""
    params = []
    for i, (fi, fo) in enumerate(zip(W.MLP_LAYERS[:-1], W.MLP_LAYERS[1:])):
        params += [W.weights(fo, fi, seed=seed0 + i), W.weights(1, fo, seed=20 + i)[0]]
    return params


def test_int8_model_chain_matches_oracle(dev):
    params = mlp_params()
    model = L.Int8Model.from_model([to_dev(p, dev) for p in params])
    assert len(model.layers) == 3
    x = W.activations(W.MLP_BATCH, W.MLP_LAYERS[0], seed=1)
    got = host(model.forward(to_dev(x, dev)))
    h = x
    for i in range(3):
        wq, sw = O.quant_rows_i8(params[2 * i])
        aq, sa = O.quant_rows_i8(h)
        h, _ = O.w8a8_linear(aq, sa, wq, sw, params[2 * i + 1], i < 2)
    np.testing.assert_array_equal(got, h)
    # mem_bytes: int8 codes + f32 row scales + f32 biases (src/int8.rs:91-93)
    n_w = sum(p.size for p in params[0::2])
    rows = sum(p.shape[0] for p in params[0::2])
    assert model.mem_bytes() == n_w + 4 * rows + 4 * sum(p.size for p in params[1::2])


def test_int8_linear_reference_forward_and_weights(dev):
    w = W.weights(48, 80, seed=3)
    b = W.weights(1, 48, seed=4)[0]
    x = W.activations(6, 80, seed=5)
    lin = L.Int8Linear.from_linear(to_dev(w, dev), to_dev(b, dev))
    wq, sw = O.quant_rows_i8(w)
    np.testing.assert_array_equal(host(lin.int8_weight.data), wq)
    np.testing.assert_array_equal(host(lin.forward(to_dev(x, dev))), O.int8_linear_forward(x, wq, sw, b))
    np.testing.assert_array_equal(host(lin.int8_weight.matmul_f32(to_dev(x, dev), 6)),
                                  O.int8_matmul_f32(wq, sw, x))
    np.testing.assert_array_equal(host(lin.int8_weight.dequantize()), O.int8_dequantize(wq, sw))
    assert lin.int8_weight.compression_ratio() == pytest.approx(48 * 80 * 4 / (48 * 80 + 4 * 48))


def test_ternary_model_from_model(dev):
    # a bias-less layer between two biased ones exercises the pairing rule
    shapes = [(64, 96), (64,), (32, 64), (16, 32), (16,)]
    params = [W.weights(*s, seed=30 + i) if len(s) == 2 else W.weights(1, s[0], seed=30 + i)[0]
              for i, s in enumerate(shapes)]
    model = L.TernaryModel.from_model([to_dev(p, dev) for p in params])
    assert [l.bias is None for l in model.layers] == [False, True, False]
    x = W.activations(5, 96, seed=7)
    t, s = O.ternary_quantize_rows(params[0])
    packed = O.pack_ternary(t)
    got = host(model.forward_first_layer(to_dev(x, dev)))
    np.testing.assert_array_equal(got, O.ternary_linear_f32(x, packed, s, 64, params[1]))
    first = model.layers[0].ternary_weight
    pos, neg, zero = first.value_counts()
    assert (pos, neg, zero) == (int((t == 1).sum()), int((t == -1).sum()), int((t == 0).sum()))
    assert first.sparsity() == zero / t.size
    # src/ternary.rs:164-166, 332-337: words + row scales (+ biases)
    exp = sum(4 * ((p.size + 15) // 16) + 4 * p.shape[0] for p in (params[0], params[2], params[3]))
    exp += 4 * (64 + 16)
    assert model.mem_bytes() == exp
    # the whole stack through the int8 ternary GEMM, ReLU between layers
    h = x
    for i, (w_i, b_i) in enumerate([(0, 1), (2, None), (3, 4)]):
        tq, ts = O.ternary_quantize_rows(params[w_i])
        aq, sa = O.quant_rows_i8(h)
        h, _ = O.ternary_gemm_i8(aq, sa, O.pack_ternary(tq), ts, params[w_i].shape[0],
                                 None if b_i is None else params[b_i], i < 2)
    np.testing.assert_array_equal(host(model.forward(to_dev(x, dev))), h)


def test_ternary_int8_forward_follows_replaced_weights(dev):
    """TernaryLinear's int8 path keeps a prepacked copy of the codes; it must
    follow `ternary_weight` when the struct is replaced (from_linear again,
    load_model) or its `packed` words are rewritten in place (the reference's
    pub fields, src/ternary.rs:81-90)."""
    import torch
    w1, w2 = W.weights(48, 256, seed=40), W.weights(48, 256, seed=41)
    x = W.activations(9, 256, seed=42)
    lin = L.TernaryLinear.from_linear(to_dev(w1, dev), None, int8=True)

    def want(w):
        t, s = O.ternary_quantize_rows(w)
        aq, sa = O.quant_rows_i8(x)
        return O.ternary_gemm_i8(aq, sa, O.pack_ternary(t), s, 48)[0]
    np.testing.assert_array_equal(host(lin.forward(to_dev(x, dev))), want(w1))
    lin.ternary_weight = L.TernaryTensor.quantize(to_dev(w2, dev))     # a new struct
    np.testing.assert_array_equal(host(lin.forward(to_dev(x, dev))), want(w2))
    t1 = L.TernaryTensor.quantize(to_dev(w1, dev))
    with torch.no_grad():                                               # the same tensor, rewritten
        lin.ternary_weight.packed.copy_(t1.packed)
        lin.ternary_weight.scales.copy_(t1.scales)
    np.testing.assert_array_equal(host(lin.forward(to_dev(x, dev))), want(w1))


@pytest.mark.parametrize("m,dims,relu", [(32, (784, 256, 128, 10), True), (1, (64, 48), False),
                                         (40, (1024, 1024, 16), True), (17, (32, 80, 112, 96, 5), True),
                                         (5, (16, 7), True),
                                         # 2, 4, 8 and 16 rows per workgroup (256 CUs)
                                         (300, (784, 256, 128, 10), True),
                                         (777, (784, 256, 128, 10), True),
                                         (1500, (128, 64, 10), True), (4111, (64, 32), False),
                                         # 4 and 8 loads of x per thread (8 and 16 rows of 1024)
                                         (1100, (1024, 32), True), (2100, (1024, 64, 10), True)])
def test_w8a8_mlp_one_launch_matches_chain(dev, hip, m, dims, relu):
    """rnn_w8a8_mlp against the oracle chain (per-row quantization + W8A8 +
    epilogue per layer, ReLU between), bit for bit; batches that give 1, 2,
    4, 8 and 16 rows of x per workgroup (the MFMAs' other rows zero; 8, 4, 2
    and 1 waves per row in the quantization pass) and 1 to 8 loads of x per
    thread, rows beyond a multiple of the workgroup's and widths that are not
    multiples of 16 included; the per-layer launches must give the same
    bits."""
    params = []
    for i, (fi, fo) in enumerate(zip(dims[:-1], dims[1:])):
        params += [W.weights(fo, fi, seed=60 + i), W.weights(1, fo, seed=70 + i)[0]]
    x = W.activations(m, dims[0], seed=80 + m)
    layers = []
    for i in range(len(dims) - 1):
        wq, sw = O.quant_rows_i8(params[2 * i])
        layers.append((to_dev(wq, dev), to_dev(sw, dev), to_dev(params[2 * i + 1], dev)))
    got = host(hip.w8a8_mlp(to_dev(x, dev), layers, relu=relu))
    h = x
    for i in range(len(dims) - 1):
        wq, sw = O.quant_rows_i8(params[2 * i])
        aq, sa = O.quant_rows_i8(h)
        h, _ = O.w8a8_linear(aq, sa, wq, sw, params[2 * i + 1], relu and i < len(dims) - 2)
    np.testing.assert_array_equal(got, h)
    model = L.Int8Model([L.Int8Linear(L.Int8Weights(w, s, w.shape), b) for w, s, b in layers])
    np.testing.assert_array_equal(host(model.forward_per_layer(to_dev(x, dev), relu)), h)


def test_w8a8_mlp_quantization_edges(dev, hip):
    """The chain's per-row quantization takes the reciprocal path with the
    exact division next to half-integers: rows whose quotients are exact
    halves (max 127 -> scale 1: 0.5, -2.5, 126.5 round away from zero), a
    row of subnormal magnitude, an all-zero row and a row with an infinity
    and a NaN must give the oracle chain's bits."""
    dims = (64, 48, 16)
    params = []
    for i, (fi, fo) in enumerate(zip(dims[:-1], dims[1:])):
        params += [W.weights(fo, fi, seed=260 + i), W.weights(1, fo, seed=270 + i)[0]]
    x = W.activations(6, dims[0], seed=281)
    x[0, :] = 0.0
    x[0, :8] = [127.0, 0.5, -2.5, 126.5, 1.5, -0.5, 63.5, -126.5]
    x[1, :] *= 1e-39                                          # subnormal scale
    x[2, :] = 0.0
    x[3, 5], x[3, 9] = np.inf, 2.0
    x[4, 7] = np.nan
    x[5, :] = np.float32(0.5) * np.arange(64, dtype=np.float32) - 16.0   # many halves
    layers, h = [], x
    for i in range(len(dims) - 1):
        wq, sw = O.quant_rows_i8(params[2 * i])
        layers.append((to_dev(wq, dev), to_dev(sw, dev), to_dev(params[2 * i + 1], dev)))
        aq, sa = O.quant_rows_i8(h)
        h, _ = O.w8a8_linear(aq, sa, wq, sw, params[2 * i + 1], i < len(dims) - 2)
    got = host(hip.w8a8_mlp(to_dev(x, dev), layers))
    np.testing.assert_array_equal(got, h)


def test_w8a8_mlp_unsupported_chains_fall_back(dev, hip):
    w = [W.weights(24, 40, seed=90), W.weights(8, 24, seed=91)]    # 40 % 16 != 0
    qs = [O.quant_rows_i8(a) for a in w]
    layers = [(to_dev(q, dev), to_dev(s, dev), None) for q, s in qs]
    x = W.activations(3, 40, seed=92)
    with pytest.raises(hip.RnnError) as e:
        hip.w8a8_mlp(to_dev(x, dev), layers)
    assert e.value.status == hip.RNN_ERR_UNSUPPORTED
    model = L.Int8Model([L.Int8Linear(L.Int8Weights(q, s, q.shape), None) for q, s, _ in layers])
    h = x
    for i, (q, s) in enumerate(qs):
        aq, sa = O.quant_rows_i8(h)
        h, _ = O.w8a8_linear(aq, sa, q, s, None, i == 0)
    np.testing.assert_array_equal(host(model.forward(to_dev(x, dev))), h)
