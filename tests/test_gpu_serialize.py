"""GPU round trip of the safetensors extension: structs quantized on the GPU
(Int8Weights, TernaryTensor, QuantizedTensor), exported, imported and rebuilt
on the device give bit-identical kernel outputs."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def test_quantized_structs_roundtrip_through_safetensors(dev, hip):
    import torch
    import layers as L
    import rnn_serialize as S
    rng = np.random.default_rng(4)
    w = torch.from_numpy((rng.standard_normal((256, 512)) * 0.02).astype(np.float32)).to(dev)
    x = torch.from_numpy(rng.standard_normal((3, 512)).astype(np.float32)).to(dev)
    i8 = L.Int8Weights.quantize(w)
    tt = L.TernaryTensor.quantize(w, hip.TERNARY_ABSMEAN)
    qt = L.QuantizedTensor.quantize(w, O.QF_GGUF_Q4, 32)
    blob = S.safetensors_export([("bias", torch.zeros(256, device=dev))],
                                [("i8", i8), ("tern", tt), ("q4", qt)])
    _, quant = S.safetensors_import(blob)
    i8b, ttb, qtb = (S.to_struct(quant[n], dev) for n in ("i8", "tern", "q4"))
    assert torch.equal(L.Int8Linear(i8).forward(x), L.Int8Linear(i8b).forward(x))
    assert torch.equal(tt.dequantize(), ttb.dequantize())
    ql, qlb = (L.QuantizedLinear(t, None, 512, 256) for t in (qt, qtb))
    assert torch.equal(ql.forward(x), qlb.forward(x))
    assert qtb.group_size == 32 and qtb.format == O.QF_GGUF_Q4
