"""Layer-level mirrors of rust-nn's quantized inference types over the HIP
library: `Int8Weights` / `Int8Linear` (src/int8.rs:11-172), `TernaryTensor` /
`TernaryLinear` / `TernaryModel` (src/ternary.rs:81-362), `QuantizedTensor` /
`QuantizedLinear` / `QuantizedModel` (src/quantize.rs:214-816), and
`Int8Model`, the int8 counterpart of `TernaryModel::from_model` that the
reference does not have.

Every tensor here is a torch device tensor; weights, codes and scales stay in
HBM for the life of a layer, and a model's forward keeps its activations on the
device between layers (quantize -> W8A8 GEMM with the ReLU fused -> quantize
...). Each method names the reference method it mirrors and calls the C ABI
through `rnn_hip`; nothing here computes on the CPU.

`from_model` takes the flat parameter list of `Module::parameters()` (weights
`[out, in]`, biases 1-D, in layer order), the reference's input to
`TernaryModel::from_model`.

`Module` mirrors the reference's layer trait (src/nn.rs:6-12), with `Linear`,
`ReLU` and `Sequential` (src/nn.rs:14-145) over the f32 kernels, so that the
quantized layers, which implement it too, sit in one `Sequential` next to f32
layers."""
from __future__ import annotations

import weakref

import rnn_hip as H


# ------------------------------------------------------------------ Module
class Module:
    """trait Module (src/nn.rs:6-12): `forward`, `parameters` (the f32 tensors
    the layer holds, in the order an optimizer or `save_model` sees them) and
    `set_training` (a no-op unless the layer behaves differently in training,
    like Dropout; every layer here is inference-only)."""

    def forward(self, x):
        raise NotImplementedError

    def parameters(self):
        return []

    def set_training(self, training):
        pass

    def __call__(self, x):
        return self.forward(x)


class Linear(Module):
    """nn::Linear (src/nn.rs:14-82): f32 `weight [out, in]` and optional
    `bias [out]`, forward through Tensor::linear_layer (rnn_linear_layer:
    x . W^T on the f32 MFMA GEMM, then + bias). Inputs of more than two
    dimensions are flattened to [leading, in] and restored, as the reference's
    N-D path does (src/nn.rs:60-78)."""

    def __init__(self, weight, bias=None):
        self.weight, self.bias = weight, bias

    def forward(self, x):
        in_f = x.shape[-1]
        lead = tuple(x.shape[:-1])
        rows = 1
        for d in lead:
            rows *= d
        y = H.linear_layer(x.reshape(rows, in_f).contiguous(), self.weight, self.bias)
        return y.reshape(*lead, self.weight.shape[0])

    def parameters(self):
        return [self.weight] + ([self.bias] if self.bias is not None else [])


class ReLU(Module):
    """nn::ReLU (src/nn.rs:134-145): Tensor::relu on the device (rnn_relu)."""

    def forward(self, x):
        return H.relu(x.contiguous())


class Sequential(Module):
    """nn::Sequential (src/nn.rs:85-132): layers applied in order; `add`
    appends and returns the model for chaining; `parameters` concatenates the
    layers' in order; `set_training` reaches every layer."""

    def __init__(self, layers=()):
        self.layers = list(layers)

    def add(self, module):
        self.layers.append(module)
        return self

    def forward(self, x):
        for layer in self.layers:
            x = layer.forward(x)
        return x

    def parameters(self):
        return [p for layer in self.layers for p in layer.parameters()]

    def set_training(self, training):
        for layer in self.layers:
            layer.set_training(training)


def pair_parameters(shapes):
    """The weight/bias pairing of `TernaryModel::from_model`
    (src/ternary.rs:291-329): a parameter is a layer's weight, and the next one
    is its bias when it is 1-D. Returns (weight index, bias index or None)
    pairs. Pure index logic over the parameter shapes, kept apart so that it
    can be checked without a GPU."""
    pairs, i = [], 0
    while i < len(shapes):
        b = i + 1 if i + 1 < len(shapes) and len(shapes[i + 1]) == 1 else None
        pairs.append((i, b))
        i += 2 if b is not None else 1
    return pairs


def _mean_abs_diff(a, b):
    # quantization_error (src/int8.rs:102-112, src/ternary.rs:174-184): mean |a - b|
    return float((a.reshape(-1) - b.reshape(-1)).abs().sum() / max(a.numel(), 1))


# ------------------------------------------------------------------ int8
class Int8Weights:
    """src/int8.rs:11-18: int8 codes `[out, in]` and one f32 scale per row."""

    def __init__(self, data, scales, shape):
        self.data, self.scales, self.shape = data, scales, tuple(shape)

    @classmethod
    def quantize(cls, weight):
        """Int8Weights::quantize (src/int8.rs:24-52)."""
        q, s = H.quant_rows_i8(weight)
        return cls(q, s, weight.shape)

    def dequantize(self):
        """Int8Weights::dequantize (src/int8.rs:55-65)."""
        return H.int8_dequantize(self.data, self.scales)

    def matmul_f32(self, activation, m):
        """Int8Weights::matmul_f32 (src/int8.rs:70-88): activation `[m, in]`."""
        return H.int8_matmul_f32(self.data, self.scales, activation.reshape(m, self.shape[1]))

    def mem_bytes(self):
        """src/int8.rs:91-93: int8 codes + f32 scales."""
        return self.data.numel() + 4 * self.scales.numel()

    def compression_ratio(self):
        """src/int8.rs:96-99."""
        return self.data.numel() * 4 / self.mem_bytes()

    def quantization_error(self, original):
        return _mean_abs_diff(original, self.dequantize())


class Int8Linear(Module):
    """src/int8.rs:117-172. `forward` keeps the reference's semantics (the
    activation quantized with the weight's row scale inside the output loop);
    `forward_w8a8` is the per-row dynamic W8A8 path of the benchmark
    configurations, with the ReLU optionally fused into the epilogue. A layer
    built with `w8a8=True` uses that path as its Module forward.
    `parameters()` is the bias: the int8 weight is frozen, not an f32 tensor."""

    def __init__(self, int8_weight, bias=None, w8a8=False):
        self.int8_weight, self.bias, self.w8a8 = int8_weight, bias, w8a8

    @classmethod
    def from_linear(cls, weight, bias=None, w8a8=False):
        """Int8Linear::from_linear (src/int8.rs:124-131)."""
        return cls(Int8Weights.quantize(weight), bias, w8a8)

    def parameters(self):
        return [self.bias] if self.bias is not None else []

    @property
    def in_features(self):
        return self.int8_weight.shape[1]

    @property
    def out_features(self):
        return self.int8_weight.shape[0]

    def forward(self, x):
        """Int8Linear::forward (src/int8.rs:134-172): x `[batch, in]`."""
        if self.w8a8:
            return self.forward_w8a8(x)
        return H.int8_linear_forward(x, self.int8_weight.data, self.int8_weight.scales, self.bias)

    def forward_w8a8(self, x, relu=False):
        """y = (Σ q(x)·W_q · sa[m]) · sw[n] + b[n], ReLU fused when asked."""
        aq, sa = H.quant_rows_i8(x)
        y, _ = H.w8a8_linear(aq, sa, self.int8_weight.data, self.int8_weight.scales, self.bias,
                             relu=relu)
        return y


class Int8Model(Module):
    """The int8 counterpart of `TernaryModel` (not in the reference): every
    weight of a parameter list quantized per row, and a device-resident forward
    that chains the W8A8 layers with the ReLU fused between them (the
    784-256-128-10 MLP of the benchmark configurations)."""

    def __init__(self, layers):
        self.layers = list(layers)

    @classmethod
    def from_model(cls, params):
        pairs = pair_parameters([tuple(p.shape) for p in params])
        return cls(Int8Linear.from_linear(params[w], None if b is None else params[b])
                   for w, b in pairs)

    def forward(self, x, relu_between=True):
        """W8A8 through every layer; ReLU after each layer but the last. Chains
        of up to 4 layers of width <= 1024 run as one launch (rnn_w8a8_mlp,
        the activation kept in LDS between layers); others launch per layer.
        Both give the same bits."""
        try:
            return H.w8a8_mlp(x.contiguous(), [(l.int8_weight.data, l.int8_weight.scales, l.bias)
                                               for l in self.layers], relu=relu_between)
        except H.RnnError as e:
            if e.status != H.RNN_ERR_UNSUPPORTED:
                raise
        return self.forward_per_layer(x, relu_between)

    def forward_per_layer(self, x, relu_between=True):
        """One quantize + W8A8 GEMM launch pair per layer."""
        for i, layer in enumerate(self.layers):
            x = layer.forward_w8a8(x, relu=relu_between and i + 1 < len(self.layers))
        return x

    def parameters(self):
        return [p for layer in self.layers for p in layer.parameters()]

    def mem_bytes(self):
        return sum(l.int8_weight.mem_bytes() + (0 if l.bias is None else 4 * l.bias.numel())
                   for l in self.layers)

    def compression_ratio(self):
        return sum(l.int8_weight.data.numel() for l in self.layers) * 4 / max(self.mem_bytes(), 1)


# ------------------------------------------------------------------ ternary
class TernaryTensor:
    """src/ternary.rs:81-90: 2-bit codes packed 16 per 32-bit word, one f32
    scale per row, the original shape and element count."""

    def __init__(self, packed, scales, shape):
        self.packed, self.scales, self.shape = packed, scales, tuple(shape)
        self.numel = self.shape[0] * self.shape[1]

    @classmethod
    def quantize(cls, tensor, mode=H.TERNARY_ROWS):
        """TernaryTensor::quantize (src/ternary.rs:97-137); `mode` =
        TERNARY_ABSMEAN selects the benchmark configuration's absmean rule."""
        packed, scales = H.ternary_quantize(tensor, mode)
        return cls(packed, scales, tensor.shape)

    def dequantize(self):
        """TernaryTensor::dequantize (src/ternary.rs:140-161)."""
        return H.ternary_dequantize(self.packed, self.numel, self.scales,
                                    self.shape[1]).reshape(self.shape)

    def mem_bytes(self):
        """src/ternary.rs:164-166: packed words + f32 scales."""
        return 4 * self.packed.numel() + 4 * self.scales.numel()

    def compression_ratio(self):
        return self.numel * 4 / max(self.mem_bytes(), 1)

    def quantization_error(self, original):
        return _mean_abs_diff(original, self.dequantize())

    def value_counts(self):
        """src/ternary.rs:194-200: counts of +1, -1 and 0."""
        t = H.ternary_unpack(self.packed, self.numel)
        return int((t == 1).sum()), int((t == -1).sum()), int((t == 0).sum())

    def sparsity(self):
        """src/ternary.rs:187-191: fraction of exact zeros."""
        return self.value_counts()[2] / max(self.numel, 1)


class TernaryLinear(Module):
    """src/ternary.rs:209-279. `forward` is the reference's sequential f32
    sum (bit-exact); `forward_int8` is the benchmark configuration's int8
    ternary GEMM over per-row quantized activations, which a layer built with
    `int8=True` uses as its Module forward. `parameters()` is the bias."""

    def __init__(self, ternary_weight, bias=None, int8=False):
        self.ternary_weight, self.bias, self.int8 = ternary_weight, bias, int8
        self.out_features, self.in_features = ternary_weight.shape

    @classmethod
    def from_linear(cls, weight, bias=None, mode=H.TERNARY_ROWS, int8=False):
        """TernaryLinear::from_linear (src/ternary.rs:218-232)."""
        return cls(TernaryTensor.quantize(weight, mode), bias, int8)

    def parameters(self):
        return [self.bias] if self.bias is not None else []

    def forward(self, x):
        """TernaryLinear::forward (src/ternary.rs:239-279): x `[batch, in]`."""
        if self.int8:
            return self.forward_int8(x)
        return H.ternary_linear_forward(x, self.ternary_weight.packed, self.ternary_weight.scales,
                                        self.out_features, self.bias)

    def forward_int8(self, x, relu=False):
        """int8 activations x 2-bit weights on int8 MFMA. When in_features %
        16 == 0 the codes are rearranged once (rnn_ternary_prepack) into the
        layout the GEMM decodes with byte permutes; the reference-layout
        `packed` field is kept as the source of truth."""
        aq, sa = H.quant_rows_i8(x)
        tw = self.ternary_weight
        if self.in_features % 16 == 0:
            # the prepacked copy follows `ternary_weight.packed`: another
            # tensor there (a replaced struct or field; held by weak reference,
            # so a freed one is never mistaken for a new one) or an in-place
            # write to it (torch's version counter) rebuilds it
            src = getattr(self, "_mfma_src", None)
            if src is None or src[0]() is not tw.packed or src[1] != tw.packed._version:
                self._mfma_packed = H.ternary_prepack(tw.packed, self.out_features,
                                                      self.in_features)
                self._mfma_src = (weakref.ref(tw.packed), tw.packed._version)
            y, _ = H.ternary_gemm(aq, sa, self._mfma_packed, tw.scales, self.out_features,
                                  self.bias, relu=relu, mfma_layout=True)
        else:
            y, _ = H.ternary_gemm(aq, sa, tw.packed, tw.scales, self.out_features, self.bias,
                                  relu=relu)
        return y


class TernaryModel(Module):
    """src/ternary.rs:285-362."""

    def __init__(self, layers):
        self.layers = list(layers)

    @classmethod
    def from_model(cls, params, mode=H.TERNARY_ROWS):
        """TernaryModel::from_model (src/ternary.rs:291-329)."""
        pairs = pair_parameters([tuple(p.shape) for p in params])
        return cls(TernaryLinear.from_linear(params[w], None if b is None else params[b], mode)
                   for w, b in pairs)

    def mem_bytes(self):
        """src/ternary.rs:332-337."""
        return sum(l.ternary_weight.mem_bytes() + (0 if l.bias is None else 4 * l.bias.numel())
                   for l in self.layers)

    def compression_ratio(self):
        """src/ternary.rs:340-344."""
        return sum(l.ternary_weight.numel for l in self.layers) * 4 / max(self.mem_bytes(), 1)

    def avg_sparsity(self):
        """src/ternary.rs:347-356."""
        if not self.layers:
            return 0.0
        return sum(l.ternary_weight.sparsity() for l in self.layers) / len(self.layers)

    def forward_first_layer(self, x):
        """src/ternary.rs:359-361."""
        return self.layers[0].forward(x)

    def forward(self, x, relu_between=True):
        """The whole stack on the device through the int8 ternary GEMM, ReLU
        fused after each layer but the last (not in the reference, which only
        runs the first layer)."""
        for i, layer in enumerate(self.layers):
            x = layer.forward_int8(x, relu=relu_between and i + 1 < len(self.layers))
        return x

    def parameters(self):
        return [p for layer in self.layers for p in layer.parameters()]


# ------------------------------------------------------------------ QuantizedTensor
QF_NAMES = {H.QF_FP16: "FP16", H.QF_BF16: "BF16", H.QF_INT8: "INT8", H.QF_INT4: "INT4",
            H.QF_NF4: "NF4 (NormalFloat 4-bit)", H.QF_NVFP4: "NVFP4 (NVIDIA FP4 E2M1)",
            H.QF_GGUF_Q4: "GGUF Q4_0", H.QF_GGUF_Q4K: "GGUF Q4_K", H.QF_GGUF_Q8: "GGUF Q8_0"}


def qf_bits(fmt):
    """QuantFormat::bits (src/quantize.rs:60-71)."""
    if fmt in (H.QF_FP16, H.QF_BF16):
        return 16
    if fmt in (H.QF_INT8, H.QF_GGUF_Q8):
        return 8
    return 4


def qf_compression_ratio(fmt):
    """QuantFormat::compression_ratio (src/quantize.rs:73-75)."""
    return 32.0 / qf_bits(fmt)


def pair_parameters_quantized(n_params):
    """The pairing of `QuantizedModel::from_model` (src/quantize.rs:758-789):
    parameter i is a weight and parameter i+1, whatever its shape, its bias;
    a trailing weight has none. Returns (weight index, bias index or None)."""
    pairs, i = [], 0
    while i < n_params:
        b = i + 1 if i + 1 < n_params else None
        pairs.append((i, b))
        i += 2 if b is not None else 1
    return pairs


class QuantizedTensor:
    """src/quantize.rs:214-227: `format`, packed `data` bytes, per-group
    `scales`, original `shape`, and the stored `group_size` (the GGUF block)."""

    def __init__(self, fmt, data, scales, shape, group_size):
        self.format, self.data, self.scales = fmt, data, scales
        self.shape, self.group_size = tuple(shape), group_size

    @classmethod
    def quantize(cls, tensor, fmt, group_size):
        """QuantizedTensor::quantize (src/quantize.rs:231-250)."""
        data, scales, g = H.qt_quantize(fmt, tensor.contiguous(), group_size)
        return cls(fmt, data, scales, tensor.shape, g)

    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def dequantize(self):
        """QuantizedTensor::dequantize (src/quantize.rs:252-269)."""
        return H.qt_dequantize(self.format, self.data, self.scales, self.group_size,
                               self.numel()).reshape(self.shape)

    def mem_bytes(self):
        """src/quantize.rs:271-274."""
        return self.data.numel() + 4 * self.scales.numel()

    def compression_ratio(self):
        """src/quantize.rs:276-280."""
        return self.numel() * 4 / self.mem_bytes()

    def quantization_error(self, original):
        """src/quantize.rs:282-293."""
        return _mean_abs_diff(original, self.dequantize())


class QuantizedLinear(Module):
    """src/quantize.rs:718-754: a quantized weight `[out, in]` and optional
    f32 bias. `forward` decodes the weight inside the GEMV (or dequantizes
    once and runs the f32 GEMM for many rows)."""

    def __init__(self, weight, bias, in_features, out_features):
        self.weight, self.bias = weight, bias
        self.in_features, self.out_features = in_features, out_features
        self._workspace = None  # the bf16 MFMA GEMV's split-K partial sums and counters, made on first use

    @classmethod
    def from_linear(cls, weight, bias, fmt, group_size):
        """QuantizedLinear::from_linear (src/quantize.rs:727-741)."""
        return cls(QuantizedTensor.quantize(weight, fmt, group_size), bias, weight.shape[1],
                   weight.shape[0])

    def forward(self, x):
        """QuantizedLinear::forward (src/quantize.rs:744-754). The layer keeps
        one workspace for the GEMV, so a forward allocates nothing but its
        output (forwards of one layer are ordered on the current stream)."""
        import torch
        w = self.weight
        if self._workspace is None:
            self._workspace = torch.zeros(H.qt_linear_workspace_size(self.in_features,
                                                                     self.out_features),
                                          dtype=torch.uint8, device=w.data.device)
        return H.qt_linear_forward(w.format, x.reshape(-1, self.in_features).contiguous(),
                                   w.data, w.scales, w.group_size, self.out_features, self.bias,
                                   workspace=self._workspace)

    def parameters(self):
        """The bias (the quantized weight is frozen, not an f32 tensor)."""
        return [self.bias] if self.bias is not None else []


class QuantizedModel:
    """src/quantize.rs:712-816."""

    def __init__(self, layers, fmt):
        self._layers, self.format = layers, fmt

    @classmethod
    def from_model(cls, params, fmt, group_size):
        """QuantizedModel::from_model (src/quantize.rs:758-789) over
        `Module::parameters()`."""
        layers = []
        for wi, bi in pair_parameters_quantized(len(params)):
            w = params[wi]
            q = QuantizedTensor.quantize(w, fmt, group_size)
            bias = None if bi is None else params[bi].reshape(-1).contiguous()
            out_f = w.shape[0] if w.dim() > 0 else 0
            in_f = w.shape[1] if w.dim() > 1 else 0
            layers.append(QuantizedLinear(q, bias, in_f, out_f))
        return cls(layers, fmt)

    def layers(self):
        return self._layers

    def mem_bytes(self):
        """src/quantize.rs:791-797."""
        return sum(l.weight.mem_bytes() + (0 if l.bias is None else 4 * l.bias.numel())
                   for l in self._layers)

    def compression_ratio(self):
        """src/quantize.rs:799-807."""
        elems = sum(l.weight.numel() for l in self._layers)
        return elems * 4 / max(self.mem_bytes(), 1)


# ------------------------------------------------------------------ RotorQuant
class RotorQuant(Module):
    """src/quant.rs:122-252: `dim`, `bits`, one Cl(3,0) rotor per 3-group
    (`rotors`, device f32 [ceil(dim/3), 4] = {s, p12, p13, p23}) and
    `padded_dim`. The rotors are given, not drawn: the reference draws them on
    the host with rand's StdRng (`new` / `with_seed`, :135-162), and the same
    values are what this layer takes. `forward` is the quantize -> dequantize
    round trip (`impl Module`, :242-252); `parameters()` is empty."""

    def __init__(self, dim, bits, rotors):
        # src/quant.rs:136 asserts bits >= 2; qmax = (1u32 << (bits - 1)) - 1
        # (:164-166) overflows past 32 bits. forward() never asks for the int8
        # codes, so widths above 8 are served too (the C ABI limits only code
        # output to 8 bits).
        if not 2 <= bits <= 32:
            raise ValueError("bits must be in [2, 32]")
        ng = (dim + 2) // 3
        if tuple(rotors.shape) != (ng, 4):
            raise ValueError(f"rotors must be [{ng}, 4], got {tuple(rotors.shape)}")
        self.dim, self.bits, self.rotors = dim, bits, rotors
        self.padded_dim = 3 * ng

    def quantize(self, x):
        """RotorQuant::quantize (src/quant.rs:212-239): any shape whose last
        dimension is `dim`."""
        if x.shape[-1] != self.dim:  # src/quant.rs:215-220
            raise ValueError(f"last dim must be {self.dim}, got {x.shape[-1]}")
        y, _, _ = H.rotorquant_quantize(x.contiguous(), self.rotors, self.bits)
        return y

    def forward(self, x):
        return self.quantize(x)
