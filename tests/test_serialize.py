"""CPU tests of rnn_serialize (src/serialize.rs): the reference's own tests,
byte-level known answers for the rnnb layout and the safetensors header, and
interoperability with the safetensors library in both directions (its
numpy loader reads what safetensors_export writes, quantized entries
included, and safetensors_import reads what its saver writes)."""
import json
import struct

import numpy as np
import pytest

import oracle as O
import rnn_serialize as S


# ----------------------------------------------------- the reference's tests
def test_serialize_deserialize_roundtrip():
    b = S.serialize([("weight", np.array([[1, 2], [3, 4]], np.float32)),
                     ("bias", np.array([5, 6], np.float32))])
    out = S.deserialize(b)
    assert [n for n, _ in out] == ["weight", "bias"]
    assert out[0][1].shape == (2, 2) and out[0][1].ravel().tolist() == [1, 2, 3, 4]


def test_save_load_model_roundtrip():
    rng = np.random.default_rng(0)
    params = [rng.standard_normal(s).astype(np.float32) for s in ((8, 4), (8,), (2, 8), (2,))]
    before = [p.copy() for p in params]
    b = S.save_model(params)
    assert b.startswith(b"RNNB")
    for p in params:
        p[...] = 0
    assert S.load_model(params, b) == 4
    assert all(np.array_equal(a, c) for a, c in zip(before, params))
    with pytest.raises(ValueError, match="parameter count mismatch"):
        S.load_model(params[:3], b)


def test_safetensors_roundtrip_empty_3d_and_names():
    t1, t2 = np.arange(1, 5, dtype=np.float32).reshape(2, 2), np.arange(5, 11, dtype=np.float32).reshape(2, 3)
    tensors, quant = S.safetensors_import(S.safetensors_export([("layer1.weight", t1),
                                                                 ("layer2.weight", t2)]))
    d = dict(tensors)
    assert not quant and np.array_equal(d["layer1.weight"], t1) and np.array_equal(d["layer2.weight"], t2)
    b = S.serialize([])
    assert b.startswith(b"RNNB") and S.deserialize(b) == []
    assert S.deserialize(S.serialize([("x", np.ones((2, 3, 4), np.float32))]))[0][1].shape == (2, 3, 4)
    tensors, _ = S.safetensors_import(S.safetensors_export([("scalar", np.array([42.0], np.float32))]))
    assert tensors[0][0] == "scalar"
    with pytest.raises(ValueError, match="invalid magic"):
        S.deserialize(b"XXXXrest of data")
    names = [n for n, _ in S.deserialize(S.save_model_named([np.zeros((5, 3), np.float32),
                                                             np.zeros(5, np.float32)],
                                                            ["weight", "bias"]))]
    assert names == ["weight", "bias"]


# ----------------------------------------------------- byte-level known answers
def test_rnnb_bytes_kat():
    """src/serialize.rs:3-16: magic, version 1, count, name_len, name, ndim,
    u64 dims, numel, little-endian f32."""
    b = S.serialize([("w", np.array([1.0, -2.0], np.float32))])
    want = (b"RNNB" + struct.pack("<III", 1, 1, 1) + b"w" + struct.pack("<I", 1) +
            struct.pack("<Q", 2) + struct.pack("<I", 2) + struct.pack("<ff", 1.0, -2.0))
    assert b == want
    with pytest.raises(ValueError, match="unsupported version"):
        S.deserialize(b"RNNB" + struct.pack("<II", 2, 0))
    with pytest.raises(ValueError, match="unexpected end"):
        S.deserialize(want[:-1])


def test_safetensors_f32_header_matches_reference_layout():
    """src/serialize.rs:164-185: entries in order, no spaces, no padding, no
    __metadata__ for f32-only exports."""
    b = S.safetensors_export([("a", np.zeros((2, 2), np.float32)), ("b", np.zeros(3, np.float32))])
    (hl,) = struct.unpack_from("<Q", b)
    assert b[8:8 + hl] == (b'{"a":{"dtype":"F32","shape":[2,2],"data_offsets":[0,16]},'
                           b'"b":{"dtype":"F32","shape":[3],"data_offsets":[16,28]}}')
    assert len(b) == 8 + hl + 28


# ----------------------------------------------------- interop with the safetensors library
def quantized_entries():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((48, 64)) * 0.02).astype(np.float32)
    q8, s8 = O.quant_rows_i8(w)
    t, g = O.ternary_quantize_absmean(w)
    packed = O.pack_ternary(t)
    d4, s4, g4 = O.qt_quantize(O.QF_INT4, w, 32)
    return w, [("l0.int8", S.QuantEntry("int8_weights", q8, s8, w.shape)),
               ("l0.ternary", S.QuantEntry("ternary", packed.view(np.uint32),
                                           np.full(48, g, np.float32), w.shape)),
               ("l0.int4", S.QuantEntry("quantized", d4, s4, w.shape, "INT4", g4))]


def test_safetensors_library_reads_our_quantized_export():
    from safetensors.numpy import load
    w, q = quantized_entries()
    b = S.safetensors_export([("l0.bias", np.arange(48, dtype=np.float32))], q)
    got = load(b)
    assert np.array_equal(got["l0.bias"], np.arange(48, dtype=np.float32))
    for name, e in q:
        assert got[f"{name}.qdata"].dtype == e.qdata.dtype
        assert np.array_equal(got[f"{name}.qdata"], e.qdata)
        assert np.array_equal(got[f"{name}.scales"], e.scales)


def test_quantized_roundtrip_and_library_written_files():
    from safetensors.numpy import save
    w, q = quantized_entries()
    tensors, quant = S.safetensors_import(S.safetensors_export([], q))
    assert tensors == [] and set(quant) == {n for n, _ in q}
    for name, e in q:
        r = quant[name]
        assert (r.kind, r.shape, r.format, r.group_size) == (e.kind, e.shape, e.format, e.group_size)
        assert np.array_equal(r.qdata, e.qdata) and np.array_equal(r.scales, e.scales)
    # the INT4 entry dequantizes to the same values
    r = quant["l0.int4"]
    assert np.array_equal(O.qt_dequantize(O.QF_INT4, r.qdata, r.scales, r.group_size, w.size),
                          O.qt_dequantize(O.QF_INT4, q[2][1].qdata, q[2][1].scales, 32, w.size))
    # a file written by the library, with its own metadata and dtypes
    meta = {"l0.int8": q[0][1].meta(), "producer": "other tool"}
    blob = save({"l0.int8.qdata": q[0][1].qdata, "l0.int8.scales": q[0][1].scales,
                 "x": np.arange(6, dtype=np.int32).reshape(2, 3)}, metadata=meta)
    tensors, quant = S.safetensors_import(blob)
    assert set(quant) == {"l0.int8"} and np.array_equal(quant["l0.int8"].qdata, q[0][1].qdata)
    assert np.array_equal(dict(tensors)["x"], np.arange(6, dtype=np.int32).reshape(2, 3))


def test_import_errors():
    with pytest.raises(ValueError, match="too short"):
        S.safetensors_import(b"1234")
    with pytest.raises(ValueError, match="exceeds"):
        S.safetensors_import(struct.pack("<Q", 100) + b"{}")
    bad = json.dumps({"__metadata__": {"q": json.dumps({"kind": "quantized", "shape": [2]})}}).encode()
    with pytest.raises(ValueError, match="missing qdata"):
        S.safetensors_import(struct.pack("<Q", len(bad)) + bad)


def test_load_model_requires_broadcastable_shapes():
    # ndarray's assign (src/serialize.rs:138): a same-size tensor of another shape
    # is an error, not a reshape; a broadcastable source fills the parameter
    b = S.save_model([np.arange(6, dtype=np.float32).reshape(2, 3)])
    with pytest.raises(ValueError, match="does not broadcast"):
        S.load_model([np.zeros((3, 2), np.float32)], b)
    with pytest.raises(ValueError, match="does not broadcast"):
        S.load_model([np.zeros(6, np.float32)], b)
    row = S.save_model([np.array([1, 2, 3], np.float32)])
    p = np.zeros((2, 3), np.float32)
    assert S.load_model([p], row) == 1
    assert p.tolist() == [[1, 2, 3], [1, 2, 3]]


def _reference_safetensors_import(data):
    """A restatement of the reference importer's control flow
    (src/serialize.rs:195-245): every header key is a tensor entry, each needs
    data_offsets, and every entry is decoded as little-endian f32."""
    (hl,) = struct.unpack_from("<Q", data, 0)
    header = json.loads(data[8:8 + hl])
    out = []
    for name, ent in header.items():
        if not isinstance(ent, dict):
            raise ValueError("entry is not an object")
        if "data_offsets" not in ent:
            raise ValueError("missing data_offsets")
        s, e = ent["data_offsets"]
        out.append((name, np.frombuffer(data[8 + hl + s:8 + hl + e][: (e - s) // 4 * 4], "<f4")))
    return out


def test_reference_importer_reads_f32_exports_but_not_quantized_ones():
    f32 = [("w", np.arange(6, dtype=np.float32).reshape(2, 3))]
    plain = S.safetensors_export(f32)
    got = _reference_safetensors_import(plain)
    assert [n for n, _ in got] == ["w"] and got[0][1].tolist() == list(range(6))
    q = S.QuantEntry("int8_weights", np.ones((2, 4), np.int8), np.ones(2, np.float32), (2, 4))
    mixed = S.safetensors_export(f32, [("layer", q)])
    with pytest.raises(ValueError, match="missing data_offsets"):
        _reference_safetensors_import(mixed)
    tensors, quant = S.safetensors_import(mixed)       # this importer reads both
    assert [n for n, _ in tensors] == ["w"] and list(quant) == ["layer"]
