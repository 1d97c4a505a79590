"""Save and load of weights for the quantized path: the reference's two
formats, kept byte for byte, and a safetensors extension for quantized
tensors (src/serialize.rs).

- `rnnb` (src/serialize.rs:3-16, :29-93): "RNNB", version u32 = 1, count u32,
  then per tensor name_len u32, name, ndim u32, dims u64[ndim], numel u32 and
  numel little-endian f32. f32 only, as in the reference, so the reference's
  `deserialize` reads what `serialize` here writes and vice versa.
- safetensors (src/serialize.rs:148-245): u64 header length, a JSON header
  mapping name -> {dtype, shape, data_offsets}, then the data. F32 tensors are
  written exactly as the reference writes them (same key order, no padding, no
  `__metadata__` when nothing is quantized). The reference cannot store its
  quantized weights at all; here a quantized tensor `name` becomes two
  standard entries, `name.qdata` (I8 for `Int8Weights::data`, U32 for
  `TernaryTensor::packed`, U8 for `QuantizedTensor::data`) and `name.scales`
  (F32), plus a `__metadata__` string describing the struct (kind, shape, and
  for `QuantizedTensor` the format and stored group size). Readers that follow
  the safetensors specification (the `safetensors` library, and
  `safetensors_import` here, which rebuilds the structs) load such files. The
  reference's own importer does not: it treats `__metadata__` as a tensor
  (Err "missing data_offsets") and reads every entry as f32 whatever its dtype
  (src/serialize.rs:209-236). A file meant for it holds f32 tensors only, which
  is what an export without quantized tensors writes, byte for byte.

Arrays are numpy; torch tensors (on any device) are accepted and copied to
the host. Host-side byte handling only: no GPU work happens here.
"""
from __future__ import annotations

import json
import struct

import numpy as np

MAGIC = b"RNNB"
VERSION = 1

# QuantFormat names (src/quantize.rs:37-56, declaration order)
QF_NAMES = ["FP16", "BF16", "INT8", "INT4", "NF4", "NVFP4", "GGUF_Q4", "GGUF_Q4K", "GGUF_Q8"]

_ST_DTYPES = {np.dtype(np.float32): "F32", np.dtype(np.int8): "I8", np.dtype(np.uint8): "U8",
              np.dtype(np.uint32): "U32", np.dtype(np.int32): "I32"}
_ST_NP = {v: k for k, v in _ST_DTYPES.items()}


def _np(a, dtype=None):
    if hasattr(a, "detach"):
        a = a.detach().cpu().numpy()
    a = np.asarray(a)
    return np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))


# ------------------------------------------------------------------ rnnb
def serialize(named):
    """serialize (src/serialize.rs:29-51): [(name, f32 array)] -> bytes."""
    out = [MAGIC, struct.pack("<II", VERSION, len(named))]
    for name, t in named:
        a = _np(t, np.float32)
        nb = name.encode("utf-8")
        out.append(struct.pack("<I", len(nb)) + nb)
        out.append(struct.pack("<I", a.ndim) + b"".join(struct.pack("<Q", d) for d in a.shape))
        out.append(struct.pack("<I", a.size) + a.astype("<f4").tobytes())
    return b"".join(out)


def deserialize(data):
    """deserialize (src/serialize.rs:55-93): bytes -> [(name, f32 array)].
    Raises ValueError where the reference returns Err."""
    data = bytes(data)
    if len(data) < 12 or data[:4] != MAGIC:
        raise ValueError("invalid magic header")
    version, count = struct.unpack_from("<II", data, 4)
    if version != VERSION:
        raise ValueError(f"unsupported version {version}")
    pos, out = 12, []

    def take(n):
        nonlocal pos
        if pos + n > len(data):
            raise ValueError("unexpected end of data")
        b = data[pos:pos + n]
        pos += n
        return b

    for _ in range(count):
        (nl,) = struct.unpack("<I", take(4))
        try:
            name = take(nl).decode("utf-8")
        except UnicodeDecodeError as e:
            raise ValueError(f"invalid name: {e}") from None
        (ndim,) = struct.unpack("<I", take(4))
        shape = [struct.unpack("<Q", take(8))[0] for _ in range(ndim)]
        (numel,) = struct.unpack("<I", take(4))
        vals = np.frombuffer(take(4 * numel), dtype="<f4").astype(np.float32)
        if int(np.prod(shape, dtype=np.int64)) != numel:
            raise ValueError("shape error: numel does not match dims")
        out.append((name, vals.reshape(shape)))
    return out


def save_model(params):
    """save_model (src/serialize.rs:96-104): parameters named param_i."""
    return serialize([(f"param_{i}", p) for i, p in enumerate(params)])


def save_model_named(params, names):
    """save_model_named (src/serialize.rs:107-122): names[i], else param_i."""
    return serialize([(names[i] if i < len(names) else f"param_{i}", p)
                      for i, p in enumerate(params)])


def load_model(params, data):
    """load_model (src/serialize.rs:125-142): copies into `params` (a list of
    numpy arrays or torch tensors, in place); returns the count."""
    loaded = deserialize(data)
    if len(loaded) != len(params):
        raise ValueError(f"parameter count mismatch: model has {len(params)}, "
                         f"checkpoint has {len(loaded)}")
    for (name, src), dst in zip(loaded, params):
        # ndarray's assign (src/serialize.rs:138) broadcasts the source to the
        # parameter's shape and panics when it cannot; a same-size tensor of
        # another shape is not reinterpreted ([2,3] into [3,2] is an error).
        try:
            view = np.broadcast_to(src, tuple(dst.shape))
        except ValueError:
            raise ValueError(f"{name}: checkpoint shape {list(src.shape)} does not broadcast to "
                             f"parameter shape {list(dst.shape)}") from None
        if hasattr(dst, "copy_"):
            import torch
            dst.copy_(torch.from_numpy(np.ascontiguousarray(view)).to(dst.device))
        else:
            dst[...] = view
    return len(loaded)


# ------------------------------------------------------------------ safetensors
class QuantEntry:
    """A quantized tensor as stored: `kind` is "int8_weights" (Int8Weights,
    src/int8.rs:11-18), "ternary" (TernaryTensor, src/ternary.rs:81-90) or
    "quantized" (QuantizedTensor, src/quantize.rs:216-227)."""

    def __init__(self, kind, qdata, scales, shape, fmt=None, group_size=None):
        self.kind, self.qdata, self.scales = kind, qdata, scales
        self.shape, self.format, self.group_size = tuple(shape), fmt, group_size

    @classmethod
    def from_struct(cls, obj):
        """From a layers.Int8Weights / TernaryTensor / QuantizedTensor."""
        name = type(obj).__name__
        if name == "Int8Weights":
            return cls("int8_weights", _np(obj.data, np.int8), _np(obj.scales, np.float32), obj.shape)
        if name == "TernaryTensor":
            return cls("ternary", _np(obj.packed).view(np.uint32), _np(obj.scales, np.float32),
                       obj.shape)
        if name == "QuantizedTensor":
            return cls("quantized", _np(obj.data, np.uint8), _np(obj.scales, np.float32), obj.shape,
                       QF_NAMES[obj.format], obj.group_size)
        raise TypeError(f"not a quantized tensor: {name}")

    def meta(self):
        m = {"kind": self.kind, "shape": list(self.shape)}
        if self.kind == "quantized":
            m["format"], m["group_size"] = self.format, self.group_size
        return json.dumps(m, separators=(",", ":"))


def _header_entry(name, dtype, shape, start, end):
    return (f"\"{name}\":{{\"dtype\":\"{dtype}\",\"shape\":[{','.join(str(int(s)) for s in shape)}],"
            f"\"data_offsets\":[{start},{end}]}}")


def safetensors_export(named, quantized=()):
    """safetensors_export (src/serialize.rs:148-192) for [(name, f32 array)],
    extended with [(name, QuantEntry or layers struct)]."""
    entries, blobs, off, meta = [], [], 0, {}

    def add(name, arr):
        nonlocal off
        a = np.ascontiguousarray(arr)
        raw = a.astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        entries.append(_header_entry(name, _ST_DTYPES[a.dtype], a.shape, off, off + len(raw)))
        blobs.append(raw)
        off += len(raw)

    for name, t in named:
        add(name, _np(t, np.float32))
    for name, q in quantized:
        q = q if isinstance(q, QuantEntry) else QuantEntry.from_struct(q)
        add(f"{name}.qdata", q.qdata)
        add(f"{name}.scales", q.scales)
        meta[name] = q.meta()
    if meta:
        md = ",".join(f"{json.dumps(k)}:{json.dumps(v)}" for k, v in meta.items())
        entries.insert(0, f"\"__metadata__\":{{{md}}}")
    header = ("{" + ",".join(entries) + "}").encode("utf-8")
    return struct.pack("<Q", len(header)) + header + b"".join(blobs)


def safetensors_import(data):
    """safetensors_import (src/serialize.rs:195-245). Returns (tensors, quant):
    `tensors` a list of (name, array) for the plain entries (F32 as the
    reference reads them; a shape [] becomes [1] as at :229-233), `quant` a
    dict name -> QuantEntry for the quantized tensors the metadata names."""
    data = bytes(data)
    if len(data) < 8:
        raise ValueError("data too short")
    (hl,) = struct.unpack_from("<Q", data, 0)
    if 8 + hl > len(data):
        raise ValueError("header length exceeds data")
    try:
        header = json.loads(data[8:8 + hl].decode("utf-8"))
    except (UnicodeDecodeError, json.JSONDecodeError) as e:
        raise ValueError(f"invalid header JSON: {e}") from None
    if not isinstance(header, dict):
        raise ValueError("header is not an object")
    meta = header.pop("__metadata__", None) or {}
    base = 8 + hl
    arrays = {}
    for name, ent in header.items():
        if not isinstance(ent, dict) or "data_offsets" not in ent:
            raise ValueError("missing data_offsets")
        s, e = ent["data_offsets"]
        dt = _ST_NP.get(ent.get("dtype"))
        if dt is None:
            raise ValueError(f"unsupported dtype {ent.get('dtype')} for {name}")
        if base + e > len(data) or s > e:
            raise ValueError("data offsets out of range")
        shape = [int(x) for x in ent.get("shape", [])] or [1]
        arrays[name] = np.frombuffer(data[base + s:base + e],
                                     dtype=dt.newbyteorder("<")).astype(dt).reshape(shape)
    quant, used = {}, set()
    for name, m in meta.items():
        try:
            info = json.loads(m)
        except (TypeError, json.JSONDecodeError):
            continue                               # foreign metadata: not ours
        if not isinstance(info, dict) or info.get("kind") not in ("int8_weights", "ternary",
                                                                  "quantized"):
            continue
        qd, sc = arrays.get(f"{name}.qdata"), arrays.get(f"{name}.scales")
        if qd is None or sc is None:
            raise ValueError(f"quantized tensor {name}: missing qdata or scales")
        quant[name] = QuantEntry(info["kind"], qd.reshape(-1) if info["kind"] != "int8_weights"
                                 else qd, sc.reshape(-1), info["shape"], info.get("format"),
                                 info.get("group_size"))
        used.update((f"{name}.qdata", f"{name}.scales"))
    tensors = [(n, a) for n, a in arrays.items() if n not in used]
    return tensors, quant


def to_struct(entry, device=None):
    """Rebuilds the layers.py struct of a QuantEntry (tensors on `device`,
    default cuda:0)."""
    import torch

    import layers as L
    dev = device or torch.device("cuda:0")

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

    if entry.kind == "int8_weights":
        return L.Int8Weights(t(entry.qdata.reshape(entry.shape)), t(entry.scales), entry.shape)
    if entry.kind == "ternary":
        return L.TernaryTensor(t(entry.qdata.view(np.int32)), t(entry.scales), entry.shape)
    return L.QuantizedTensor(QF_NAMES.index(entry.format), t(entry.qdata), t(entry.scales),
                             entry.shape, entry.group_size)
