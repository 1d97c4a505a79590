"""CPU check of the weight/bias pairing that `TernaryModel::from_model`
(src/ternary.rs:291-329) applies to `Module::parameters()`, as mirrored by
`layers.pair_parameters` for TernaryModel and Int8Model."""
import layers as L


def test_pairs_weights_with_following_1d_bias():
    # Sequential(Linear(784,256), ReLU, Linear(256,128), ReLU, Linear(128,10))
    shapes = [(256, 784), (256,), (128, 256), (128,), (10, 128), (10,)]
    assert L.pair_parameters(shapes) == [(0, 1), (2, 3), (4, 5)]


def test_pairs_without_bias_and_trailing_weight():
    # a 2-D parameter after a weight is the next layer's weight, not a bias;
    # a final weight with nothing after it is a layer of its own
    assert L.pair_parameters([(4, 3), (5, 4), (5,), (2, 5)]) == [(0, None), (1, 2), (3, None)]
    assert L.pair_parameters([(4, 3)]) == [(0, None)]
    assert L.pair_parameters([]) == []


def test_a_leading_1d_parameter_is_taken_as_a_weight():
    # the reference treats parameter i as a weight whatever its rank
    assert L.pair_parameters([(3,), (3,), (2, 3)]) == [(0, 1), (2, None)]


def test_quantized_model_pairing():
    """QuantizedModel::from_model (src/quantize.rs:762-787) takes parameter
    i+1 as the bias of weight i whatever its shape, stepping by two; a
    trailing weight has no bias."""
    from layers import pair_parameters_quantized as P
    assert P(4) == [(0, 1), (2, 3)]
    assert P(3) == [(0, 1), (2, None)]
    assert P(1) == [(0, None)]
    assert P(0) == []
