"""GPU parity of the Module mirrors (trait Module, src/nn.rs:6-12): a
Sequential (src/nn.rs:85-132) that mixes the quantized layers with ReLU and an
f32 Linear, against the oracle chain on the same inputs; and the f32 pieces
it needs on their own -- Tensor::relu, linear_layer's fused bias + ReLU and
linear_layer itself (src/tensor.rs:747-800, :2025-2032).

Tolerances: the quantized layers and ReLU are bit-exact; an f32 Linear sums in
the MFMA GEMM's own order, so it is held to the rnn_sgemm rounding bound
|err| <= gamma_(k+2) * (|x||W|^T + |b|) of a float64 product."""
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


def linear_bound(x, w, b):
    k = x.shape[-1]
    u = 2.0 ** -24
    g = (k + 2) * u / (1 - (k + 2) * u)
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    return g * (mag + (0 if b is None else np.abs(b.astype(np.float64)))) + 1e-30


def linear_f64(x, w, b):
    y = x.astype(np.float64) @ w.astype(np.float64).T
    return y if b is None else y + b.astype(np.float64)


def test_mixed_sequential_matches_oracle_chain(dev):
    """Int8Linear (reference forward) -> ReLU -> TernaryLinear (reference f32
    forward) -> ReLU -> Int8Linear (W8A8 path) -> ReLU -> Linear (f32)."""
    w1, b1 = W.weights(256, 784, seed=40), W.weights(1, 256, seed=41)[0]
    w2, b2 = W.weights(128, 256, seed=42), W.weights(1, 128, seed=43)[0]
    w3, b3 = W.weights(64, 128, seed=44), W.weights(1, 64, seed=45)[0]
    w4, b4 = W.weights(10, 64, seed=46, std=0.2), W.weights(1, 10, seed=47)[0]
    seq = (L.Sequential()
           .add(L.Int8Linear.from_linear(to_dev(w1, dev), to_dev(b1, dev)))
           .add(L.ReLU())
           .add(L.TernaryLinear.from_linear(to_dev(w2, dev), to_dev(b2, dev)))
           .add(L.ReLU())
           .add(L.Int8Linear.from_linear(to_dev(w3, dev), to_dev(b3, dev), w8a8=True))
           .add(L.ReLU())
           .add(L.Linear(to_dev(w4, dev), to_dev(b4, dev))))
    x = W.activations(W.MLP_BATCH, 784, seed=48)
    got = host(seq.forward(to_dev(x, dev)))

    q1, s1 = O.quant_rows_i8(w1)
    h = O.relu(O.int8_linear_forward(x, q1, s1, b1))
    t2, s2 = O.ternary_quantize_rows(w2)
    h = O.relu(O.ternary_linear_f32(h, O.pack_ternary(t2), s2, 128, b2))
    q3, s3 = O.quant_rows_i8(w3)
    aq, sa = O.quant_rows_i8(h)
    h, _ = O.w8a8_linear(aq, sa, q3, s3, b3, relu=True)
    # every layer up to here is bit-exact, so the f32 Linear sees the oracle's input
    np.testing.assert_array_equal(host(seq.layers[5].forward(seq.layers[4].forward(
        seq.layers[3].forward(seq.layers[2].forward(seq.layers[1].forward(
            seq.layers[0].forward(to_dev(x, dev)))))))), h)
    assert np.all(np.abs(got - linear_f64(h, w4, b4)) <= linear_bound(h, w4, b4))
    # parameters(): the biases of the quantized layers, then Linear's weight and bias
    ps = seq.parameters()
    assert len(ps) == 5 and ps[3] is seq.layers[6].weight
    np.testing.assert_array_equal(host(ps[0]), b1)


def test_sequential_quantized_linear_and_rotorquant(dev):
    """QuantizedLinear (INT4 g64) -> ReLU, and a RotorQuant round trip as a
    Module (src/quant.rs:242-252), inside one Sequential."""
    w = W.weights(96, 128, seed=50)
    x = W.activations(8, 128, seed=51)
    rot = W.rotors(43, seed=52)
    ql = L.QuantizedLinear.from_linear(to_dev(w, dev), None, O.QF_INT4, 64)
    seq = L.Sequential([L.RotorQuant(128, 4, to_dev(rot, dev)), ql, L.ReLU()])
    got = host(seq.forward(to_dev(x, dev)))
    xq, _, _ = O.rotorquant_quantize(x, rot, 4)
    d, s, g = O.qt_quantize(O.QF_INT4, w, 64)
    wd = O.qt_dequantize(O.QF_INT4, d, s, g, w.size).reshape(w.shape)
    ref = linear_f64(xq, wd, None)
    bound = linear_bound(xq, wd, None)
    # ReLU of a value within the bound of ref stays within the bound of relu(ref)
    assert np.all(np.abs(got - np.maximum(ref, 0)) <= bound)
    assert seq.parameters() == []


@pytest.mark.parametrize("bits", [12, 16])
def test_rotorquant_module_wide_codes(dev, bits):
    """RotorQuant::new(dim, bits) with bits above 8 (src/quant.rs:135-166):
    the Module round trip, bit for bit against the oracle."""
    x = W.activations(200, 128, seed=60 + bits)
    rot = W.rotors(43, seed=62)
    got = host(L.RotorQuant(128, bits, to_dev(rot, dev)).forward(to_dev(x, dev)))
    want, _, _ = O.rotorquant_quantize(x, rot, bits)
    np.testing.assert_array_equal(got, want)


def test_relu_matches_f32_max(dev, hip):
    x = W.activations(7, 333, seed=53)
    x[0, :4] = [np.nan, -0.0, 0.0, -np.inf]
    got = host(hip.relu(to_dev(x, dev)))
    np.testing.assert_array_equal(got, O.relu(x))
    # unaligned tail and in-place use
    xd = to_dev(x.reshape(-1), dev)
    hip.relu(xd[1:], out=xd[1:])
    np.testing.assert_array_equal(host(xd)[1:], O.relu(x.reshape(-1)[1:]))


@pytest.mark.parametrize("rows,cols,relu", [(5, 64, False), (5, 64, True), (3, 37, True)])
def test_bias_act_matches_linear_layer_loop(dev, hip, rows, cols, relu):
    y = W.activations(rows, cols, seed=54)
    b = W.activations(1, cols, seed=55)[0]
    y[0, 0] = np.nan
    exp = (y + b[None, :]).astype(np.float32)   # one f32 rounding per add
    if relu:
        exp = np.where(exp > 0, exp, np.float32(0.0)).astype(np.float32)  # NaN -> 0 as well
    got = host(hip.bias_act(to_dev(y, dev), to_dev(b, dev), relu=relu))
    np.testing.assert_array_equal(got, exp)


@pytest.mark.parametrize("batch,in_f,out_f,bias,relu",
                         [(32, 784, 256, True, False), (7, 130, 33, True, True),
                          (1, 64, 10, False, False), (5, 0, 6, True, False)])
def test_linear_layer_within_gemm_bound(dev, hip, batch, in_f, out_f, bias, relu):
    x = W.activations(batch, in_f, seed=56)
    w = W.weights(out_f, in_f, seed=57, std=0.1)
    b = W.weights(1, out_f, seed=58)[0] if bias else None
    got = host(hip.linear_layer(to_dev(x, dev), to_dev(w, dev),
                                None if b is None else to_dev(b, dev), relu=relu))
    ref = linear_f64(x, w, b)
    if relu:
        ref = np.maximum(ref, 0)
    assert np.all(np.abs(got - ref) <= linear_bound(x, w, b))
    # the N-D path of Linear::forward (src/nn.rs:60-78): [2, batch, in] -> [2, batch, out]
    lin = L.Linear(to_dev(w, dev), None if b is None else to_dev(b, dev))
    x3 = np.stack([x, x])
    y3 = host(lin.forward(to_dev(x3, dev)))
    assert y3.shape == (2, batch, out_f)
    np.testing.assert_array_equal(y3[1], host(lin.forward(to_dev(x, dev))))
