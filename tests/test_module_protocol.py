"""The Module protocol of the layer mirrors (trait Module, src/nn.rs:6-12;
Sequential src/nn.rs:85-132) as host logic: parameter order, chaining,
set_training propagation and which tensors each quantized layer reports.
No GPU: the layers are built around stand-in tensors and stub modules."""
import layers as L


class _Probe(L.Module):
    def __init__(self, tag, params=()):
        self.tag, self._params, self.training = tag, list(params), None

    def forward(self, x):
        return x + [self.tag]

    def parameters(self):
        return list(self._params)

    def set_training(self, training):
        self.training = training


def test_sequential_chains_in_order_and_collects_parameters():
    a, b, c = _Probe("a", ["wa", "ba"]), _Probe("b"), _Probe("c", ["wc"])
    seq = L.Sequential().add(a).add(b).add(c)   # add returns the model (src/nn.rs:95-99)
    assert seq.forward([]) == ["a", "b", "c"]
    assert seq([]) == ["a", "b", "c"]
    assert seq.parameters() == ["wa", "ba", "wc"]
    seq.set_training(False)
    assert (a.training, b.training, c.training) == (False, False, False)
    nested = L.Sequential([seq, _Probe("d", ["wd"])])
    assert nested.forward([]) == ["a", "b", "c", "d"]
    assert nested.parameters() == ["wa", "ba", "wc", "wd"]


def test_layers_report_their_f32_tensors():
    # nn::Linear: weight then bias (src/nn.rs:84-90); ReLU and RotorQuant: none
    assert L.Linear("W", "b").parameters() == ["W", "b"]
    assert L.Linear("W").parameters() == ["W"]
    assert L.ReLU().parameters() == []
    # quantized layers hold a frozen weight; only the f32 bias is a parameter
    w8 = L.Int8Weights("codes", "scales", (4, 8))
    assert L.Int8Linear(w8, "bias").parameters() == ["bias"]
    assert L.Int8Linear(w8).parameters() == []

    class _T:  # TernaryTensor stand-in: only the shape is read at construction
        shape = (4, 8)
    assert L.TernaryLinear(_T(), "bias").parameters() == ["bias"]
    assert L.QuantizedLinear("qt", None, 8, 4).parameters() == []
    m = L.Int8Model([L.Int8Linear(w8, "b1"), L.Int8Linear(w8), L.Int8Linear(w8, "b3")])
    assert m.parameters() == ["b1", "b3"]
    for layer in (L.Linear("W"), L.ReLU(), L.Int8Linear(w8), L.TernaryLinear(_T())):
        assert isinstance(layer, L.Module)
        layer.set_training(True)  # the default is a no-op (src/nn.rs:11)


def test_rotorquant_module_checks_its_arguments():
    import pytest

    class _R:
        shape = (43, 4)
    rq = L.RotorQuant(128, 4, _R())
    assert rq.padded_dim == 129 and rq.parameters() == []
    with pytest.raises(ValueError):
        L.RotorQuant(128, 1, _R())      # at least 2 bits (src/quant.rs:136)
    with pytest.raises(ValueError):
        L.RotorQuant(128, 33, _R())     # qmax's u32 shift (src/quant.rs:164-166)
    assert L.RotorQuant(128, 16, _R()).bits == 16   # RotorQuant::new(dim, 16) is valid
    with pytest.raises(ValueError):
        L.RotorQuant(126, 4, _R())      # 42 groups need 42 rotors
