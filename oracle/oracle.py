"""numpy front-end for the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP kernels and the CPU
baseline timed by bench.py. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module. Every function restates a reference
function of gugu8intel-i9/Rust-Neural-Network; the citation is in oracle.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


def build() -> None:
    """Compile liboracle.so with oracle/Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-B", "-C", _HERE, "liboracle.so"], check=True,
                   stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        sig = {
            "orc_lcg_bytes": [_P, _P, _SZ, ctypes.c_int],
            "orc_igemm_scalar": [_P, _P, _P, _SZ, _SZ, _SZ],
            "orc_igemm": [_P, _P, _P, _SZ, _SZ, _SZ, ctypes.c_int],
            "orc_quant_rows_i8": [_P, _SZ, _SZ, _P, _P],
            "orc_int8_dequantize": [_P, _P, _SZ, _SZ, _P],
            "orc_int8_matmul_f32": [_P, _P, _SZ, _SZ, _P, _SZ, _P],
            "orc_int8_linear_forward": [_P, _SZ, _SZ, _P, _P, _SZ, _P, _P],
            "orc_w8a8_linear": [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, ctypes.c_int, _P, _P],
            "orc_relu": [_P, _SZ],
            "orc_pack_ternary": [_P, _SZ, _P],
            "orc_unpack_ternary": [_P, _SZ, _P],
            "orc_ternary_quantize_rows": [_P, _SZ, _SZ, _P, _P],
            "orc_ternary_quantize_absmean": [_P, _SZ, _SZ, _P],
            "orc_ternary_dequantize": [_P, _SZ, _P, _SZ, _SZ, _P],
            "orc_ternary_linear_f32": [_P, _SZ, _SZ, _P, _P, _SZ, _P, _P],
            "orc_ternary_gemm_i8": [_P, _P, _P, _P, _P, _SZ, _SZ, _SZ, ctypes.c_int, _P, _P],
            "orc_rotor_sandwich": [_P, _P, _P],
            "orc_rotor_inv_sandwich": [_P, _P, _P],
            "orc_rotor_rotation_matrix": [_P, _P],
            "orc_rotorquant_quantize": [_P, _SZ, _SZ, ctypes.c_int, _P, _P, _P, _P],
            "orc_rotorquant_dequantize": [_P, _P, _SZ, _SZ, _P, _P],
            "orc_f32_to_f16": [ctypes.c_float],
            "orc_f16_to_f32": [ctypes.c_uint16],
            "orc_f32_to_bf16": [ctypes.c_float],
            "orc_bf16_to_f32": [ctypes.c_uint16],
            "orc_f32_to_f16_array": [_P, _SZ, _P],
            "orc_f16_to_f32_array": [_P, _SZ, _P],
            "orc_f32_to_bf16_array": [_P, _SZ, _P],
            "orc_bf16_to_f32_array": [_P, _SZ, _P],
            "orc_qt_layout": [ctypes.c_int, _SZ, _SZ, _P, _P],
            "orc_qt_quantize": [ctypes.c_int, _P, _SZ, _SZ, _P, _P],
            "orc_qt_dequantize": [ctypes.c_int, _P, _P, _SZ, _SZ, _SZ, _P],
            "orc_qt_linear_forward": [ctypes.c_int, _P, _SZ, _SZ, _P, _P, _SZ, _SZ, _SZ, _P, _P],
            "orc_flash_attention": [_P, _P, _P, _SZ, _SZ, _SZ, _SZ, ctypes.c_float, _P],
            "orc_sgemm": [ctypes.c_int, ctypes.c_int, _SZ, _SZ, _SZ, ctypes.c_float, _P, _SZ, _P, _SZ,
                          ctypes.c_float, _P, _SZ],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = None
        L.orc_igemm.restype = ctypes.c_int
        L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_f16_to_f32.restype = ctypes.c_float
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_bf16_to_f32.restype = ctypes.c_float
        L.orc_qt_layout.restype = _SZ
        L.orc_ternary_quantize_absmean.restype = ctypes.c_float
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a):
    return None if a is None else a.ctypes.data


# ---------------------------------------------------------------- generators
def lcg_bytes(seed: int, n: int, signed: bool):
    """src/int8.rs:382-394. Returns (bytes as int8, next seed)."""
    s = (ctypes.c_uint32 * 1)(seed)
    out = np.empty(n, np.int8)
    lib().orc_lcg_bytes(ctypes.addressof(s), _ptr(out), n, int(signed))
    return out, int(s[0])


# ---------------------------------------------------------------- int8
def igemm_scalar(a_u8, b_i8, m, k, n):
    a, b = _c(a_u8, np.uint8), _c(b_i8, np.int8)
    c = np.empty((m, n), np.int32)
    lib().orc_igemm_scalar(_ptr(a), _ptr(b), _ptr(c), m, k, n)
    return c


def igemm(a_u8, b_i8, m, k, n, nthreads=1):
    """src/int8.rs:285-314. Returns (C, used_vnni)."""
    a, b = _c(a_u8, np.uint8), _c(b_i8, np.int8)
    c = np.empty((m, n), np.int32)
    used = lib().orc_igemm(_ptr(a), _ptr(b), _ptr(c), m, k, n, nthreads)
    return c, bool(used)


def quant_rows_i8(x):
    x = _c(x, np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_quant_rows_i8(_ptr(x), rows, cols, _ptr(q), _ptr(s))
    return q, s


def int8_dequantize(q, s):
    q, s = _c(q, np.int8), _c(s, np.float32)
    w = np.empty(q.shape, np.float32)
    lib().orc_int8_dequantize(_ptr(q), _ptr(s), q.shape[0], q.shape[1], _ptr(w))
    return w


def int8_matmul_f32(wq, ws, x):
    wq, ws, x = _c(wq, np.int8), _c(ws, np.float32), _c(x, np.float32)
    out_f, in_f = wq.shape
    m = x.size // in_f
    y = np.empty((m, out_f), np.float32)
    lib().orc_int8_matmul_f32(_ptr(wq), _ptr(ws), out_f, in_f, _ptr(x), m, _ptr(y))
    return y


def int8_linear_forward(x, wq, ws, bias=None):
    x, wq, ws = _c(x, np.float32), _c(wq, np.int8), _c(ws, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    batch, in_f = x.shape
    out_f = wq.shape[0]
    y = np.empty((batch, out_f), np.float32)
    lib().orc_int8_linear_forward(_ptr(x), batch, in_f, _ptr(wq), _ptr(ws), out_f,
                                  _ptr(bias), _ptr(y))
    return y


def w8a8_linear(aq, sa, wq, sw, bias=None, relu=False):
    """Returns (y f32 [m,n], acc int32 [m,n])."""
    aq, sa, wq, sw = _c(aq, np.int8), _c(sa, np.float32), _c(wq, np.int8), _c(sw, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    m, k = aq.shape
    n = wq.shape[0]
    y = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32)
    lib().orc_w8a8_linear(_ptr(aq), _ptr(sa), _ptr(wq), _ptr(sw), _ptr(bias), m, k, n,
                          int(relu), _ptr(y), _ptr(acc))
    return y, acc


def relu(x):
    y = _c(x, np.float32).copy()
    lib().orc_relu(_ptr(y), y.size)
    return y


# ---------------------------------------------------------------- ternary
def pack_ternary(v):
    v = _c(v, np.int8).ravel()
    out = np.empty((v.size + 15) // 16, np.uint32)
    lib().orc_pack_ternary(_ptr(v), v.size, _ptr(out))
    return out


def unpack_ternary(packed, count):
    p = _c(packed, np.uint32)
    out = np.empty(count, np.int8)
    lib().orc_unpack_ternary(_ptr(p), count, _ptr(out))
    return out


def ternary_quantize_rows(w):
    w = _c(w, np.float32)
    rows, cols = w.shape if w.ndim == 2 else (1, w.size)
    t = np.empty(rows * cols, np.int8)
    s = np.empty(rows, np.float32)
    lib().orc_ternary_quantize_rows(_ptr(w), rows, cols, _ptr(t), _ptr(s))
    return t.reshape(w.shape), s


def ternary_quantize_absmean(w):
    w = _c(w, np.float32)
    rows, cols = w.shape
    t = np.empty((rows, cols), np.int8)
    g = lib().orc_ternary_quantize_absmean(_ptr(w), rows, cols, _ptr(t))
    return t, np.float32(g)


def ternary_dequantize(packed, numel, scales, cols):
    p, s = _c(packed, np.uint32), _c(scales, np.float32)
    w = np.empty(numel, np.float32)
    lib().orc_ternary_dequantize(_ptr(p), numel, _ptr(s), s.size, cols, _ptr(w))
    return w


def ternary_linear_f32(x, packed, scales, out_f, bias=None):
    x, p, s = _c(x, np.float32), _c(packed, np.uint32), _c(scales, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    batch, in_f = x.shape
    y = np.empty((batch, out_f), np.float32)
    lib().orc_ternary_linear_f32(_ptr(x), batch, in_f, _ptr(p), _ptr(s), out_f,
                                 _ptr(bias), _ptr(y))
    return y


def ternary_gemm_i8(aq, sa, packed, sw, n, bias=None, relu=False):
    aq, sa, p, sw = _c(aq, np.int8), _c(sa, np.float32), _c(packed, np.uint32), _c(sw, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    m, k = aq.shape
    y = np.empty((m, n), np.float32)
    acc = np.empty((m, n), np.int32)
    lib().orc_ternary_gemm_i8(_ptr(aq), _ptr(sa), _ptr(p), _ptr(sw), _ptr(bias), m, k, n,
                              int(relu), _ptr(y), _ptr(acc))
    return y, acc


# ---------------------------------------------------------------- rotors
def rotor_sandwich(r, x, inverse=False):
    r, x = _c(r, np.float32), _c(x, np.float32)
    out = np.empty(8, np.float32)
    fn = lib().orc_rotor_inv_sandwich if inverse else lib().orc_rotor_sandwich
    fn(_ptr(r), _ptr(x), _ptr(out))
    return out


def rotor_rotation_matrix(r):
    r = _c(r, np.float32)
    out = np.empty(9, np.float32)
    lib().orc_rotor_rotation_matrix(_ptr(r), _ptr(out))
    return out.reshape(3, 3)


def rotorquant_quantize(x, rotors, bits):
    """src/quant.rs:212-239. Returns (y, codes [rows,padded], scales [rows,groups])."""
    x, r = _c(x, np.float32), _c(rotors, np.float32)
    dim = x.shape[-1]
    rows = x.size // dim
    padded = (dim + 2) // 3 * 3
    y = np.empty(x.shape, np.float32)
    codes = np.empty((rows, padded), np.int8)
    scales = np.empty((rows, padded // 3), np.float32)
    lib().orc_rotorquant_quantize(_ptr(x), rows, dim, bits, _ptr(r), _ptr(y),
                                  _ptr(codes), _ptr(scales))
    return y, codes, scales


def rotorquant_dequantize(codes, scales, dim, rotors):
    c, s, r = _c(codes, np.int8), _c(scales, np.float32), _c(rotors, np.float32)
    rows = c.shape[0]
    y = np.empty((rows, dim), np.float32)
    lib().orc_rotorquant_dequantize(_ptr(c), _ptr(s), rows, dim, _ptr(r), _ptr(y))
    return y


# ---------------------------------------------------------------- f32 GEMM
def sgemm(transa, transb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc):
    """src/blas.rs:104-264 (gemm_small order): returns the updated copy of c
    (flat f32 storage with row stride ldc)."""
    a = _c(a, np.float32).ravel()
    b = _c(b, np.float32).ravel()
    out = _c(c, np.float32).ravel().copy()
    lib().orc_sgemm(int(transa), int(transb), m, n, k, float(alpha), _ptr(a), lda, _ptr(b), ldb,
                    float(beta), _ptr(out), ldc)
    return out


def blas_rand_mat(seed: int, n: int):
    """The reference's sgemm test generator (src/blas.rs tests, rand_mat):
    s = s*1664525 + 1013904223 (mod 2^32), value = (s >> 8) / 2^24 - 0.5.
    Returns (values f32 [n], next seed)."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32(np.float32(s >> 8) / np.float32(16777216.0)) - np.float32(0.5)
    return out, s


# (name, transa, transb, m, n, k, seed, alpha, beta, tolerance of the reference's test)
# from the reference's sgemm tests (src/blas.rs:1195-1512)
BLAS_TEST_CASES = [
    ("nn", 0, 0, 17, 19, 13, 1, 1.0, 0.0, 1e-3),
    ("nt", 0, 1, 33, 29, 17, 2, 1.0, 0.0, 1e-3),
    ("tn", 1, 0, 29, 33, 17, 3, 1.0, 0.0, 1e-3),
    ("tt", 1, 1, 40, 35, 24, 4, 1.0, 0.0, 1e-3),
    ("alpha_beta", 0, 0, 20, 20, 20, 5, 2.5, -1.5, 1e-3),
    ("large_blocked", 0, 0, 200, 180, 160, 6, 1.0, 0.0, 0.1),
]


def blas_test_case(transa, transb, m, n, k, seed, beta):
    """Operands of one BLAS_TEST_CASES entry, drawn in the reference's order
    (A, then B, then C when beta != 0) with its storage shapes and leading
    dimensions. Returns (a, lda, b, ldb, c0)."""
    a, s = blas_rand_mat(seed, m * k)
    b, s = blas_rand_mat(s, k * n)
    c0 = blas_rand_mat(s, m * n)[0] if beta != 0.0 else np.zeros(m * n, np.float32)
    lda = m if transa else k
    ldb = k if transb else n
    return a, lda, b, ldb, c0


def sgemm_f64(transa, transb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc):
    """The exact value in float64 and the rounding scale
    |alpha| * (|op(A)| |op(B)|) + |beta C|, both [m, n]."""
    def op(x, ld, rows, cols, trans):
        # the logical [rows, cols] operand of storage x with row stride ld
        x = np.asarray(x, np.float64).ravel()
        if trans:  # stored [cols, rows]
            return np.lib.stride_tricks.as_strided(x, shape=(cols, rows), strides=(ld * 8, 8)).T
        return np.lib.stride_tricks.as_strided(x, shape=(rows, cols), strides=(ld * 8, 8))
    A = op(a, lda, m, k, transa)
    B = op(b, ldb, k, n, transb)
    C = np.lib.stride_tricks.as_strided(np.asarray(c, np.float64).ravel(), shape=(m, n), strides=(ldc * 8, 8))
    exact = alpha * (A @ B) + (beta * C if beta != 0.0 else 0.0)
    scale = abs(alpha) * (np.abs(A) @ np.abs(B)) + (abs(beta) * np.abs(C) if beta != 0.0 else 0.0)
    return exact, scale


# ---------------------------------------------------------------- QuantizedTensor
# QuantFormat (src/quantize.rs:37-56), declaration order
QF_FP16, QF_BF16, QF_INT8, QF_INT4, QF_NF4, QF_NVFP4, QF_GGUF_Q4, QF_GGUF_Q4K, QF_GGUF_Q8 = range(9)
QF_NAMES = {QF_FP16: "FP16", QF_BF16: "BF16", QF_INT8: "INT8", QF_INT4: "INT4", QF_NF4: "NF4",
            QF_NVFP4: "NVFP4", QF_GGUF_Q4: "GGUF_Q4", QF_GGUF_Q4K: "GGUF_Q4K",
            QF_GGUF_Q8: "GGUF_Q8"}
# QuantFormat::bits (src/quantize.rs:60-71)
QF_BITS = {QF_FP16: 16, QF_BF16: 16, QF_INT8: 8, QF_GGUF_Q8: 8, QF_INT4: 4, QF_NF4: 4,
           QF_NVFP4: 4, QF_GGUF_Q4: 4, QF_GGUF_Q4K: 4}


def _conv(name, x, in_dtype, out_dtype):
    x = _c(x, in_dtype).ravel()
    out = np.empty(x.size, out_dtype)
    getattr(lib(), name)(_ptr(x), x.size, _ptr(out))
    return out


def f32_to_f16(x):
    """src/quantize.rs:639-666 over an array (uint16 bit patterns)."""
    return _conv("orc_f32_to_f16_array", x, np.float32, np.uint16)


def f16_to_f32(h):
    """src/quantize.rs:668-695 over an array."""
    return _conv("orc_f16_to_f32_array", h, np.uint16, np.float32)


def f32_to_bf16(x):
    """src/quantize.rs:697-703 over an array."""
    return _conv("orc_f32_to_bf16_array", x, np.float32, np.uint16)


def bf16_to_f32(h):
    """src/quantize.rs:705-708 over an array."""
    return _conv("orc_bf16_to_f32_array", h, np.uint16, np.float32)


def qt_layout(fmt, n, group_size):
    """(data bytes, scales.len(), stored group_size) of QuantizedTensor::quantize."""
    ns, g = (ctypes.c_size_t * 1)(), (ctypes.c_size_t * 1)()
    nb = lib().orc_qt_layout(fmt, n, group_size, ctypes.addressof(ns), ctypes.addressof(g))
    return int(nb), int(ns[0]), int(g[0])


def qt_quantize(fmt, x, group_size):
    """QuantizedTensor::quantize (src/quantize.rs:231-250). Returns
    (data uint8, scales f32, stored group_size)."""
    x = _c(x, np.float32).ravel()
    nb, ns, g = qt_layout(fmt, x.size, group_size)
    data = np.zeros(nb, np.uint8)
    scales = np.zeros(ns, np.float32)
    lib().orc_qt_quantize(fmt, _ptr(x), x.size, group_size, _ptr(data), _ptr(scales))
    return data, scales, g


def qt_dequantize(fmt, data, scales, group, n):
    """QuantizedTensor::dequantize (src/quantize.rs:252-269), flat f32 [n]."""
    data, scales = _c(data, np.uint8), _c(scales, np.float32)
    out = np.empty(n, np.float32)
    lib().orc_qt_dequantize(fmt, _ptr(data), _ptr(scales), scales.size, group, n, _ptr(out))
    return out


def qt_linear_forward(fmt, x, data, scales, group, out_f, bias=None):
    """QuantizedLinear::forward (src/quantize.rs:744-754)."""
    x, data, scales = _c(x, np.float32), _c(data, np.uint8), _c(scales, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    m, in_f = x.shape
    y = np.empty((m, out_f), np.float32)
    lib().orc_qt_linear_forward(fmt, _ptr(x), m, in_f, _ptr(data), _ptr(scales), scales.size,
                                group, out_f, _ptr(bias), _ptr(y))
    return y


# ---------------------------------------------------------------- attention
def flash_attention(q, k, v, scale):
    """Tensor::flash_attention (src/tensor.rs:618-672): q [batch, nq, dim],
    k, v [batch, skv, dim] (nq == skv is the reference's signature)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    b, nq, dim = q.shape
    skv = k.shape[1]
    out = np.empty((b, nq, dim), np.float32)
    lib().orc_flash_attention(_ptr(q), _ptr(k), _ptr(v), b, nq, skv, dim, float(scale), _ptr(out))
    return out
