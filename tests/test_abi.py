"""CPU-only checks of the C ABI: the library loads, exports every symbol that
include/rnn_hip.h declares, and rejects bad arguments before touching a GPU
(the reference panics on these; the ABI returns a status code instead)."""
import ctypes
import os
import subprocess

import pytest

import rnn_hip as H

FAKE = ctypes.c_void_p(256)  # never dereferenced: every case fails validation first


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(H.LIB_PATH):
        import build as B
        B.build()
    return H.load()


def test_header_symbols_are_exported(lib):
    names = H.header_symbols()
    assert len(names) >= 18
    out = subprocess.run(["nm", "-D", "--defined-only", H.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    assert sorted(H.SIGNATURES) == names  # the binding covers the whole header


def test_abi_version(lib):
    assert lib.rnn_abi_version() == 1


def _status(rc, code, needle):
    assert rc == code, H.last_error()
    assert needle in H.last_error()


def test_negative_sizes_rejected(lib):
    _status(lib.rnn_quant_rows_i8(FAKE, -1, 4, FAKE, FAKE, None), H.RNN_ERR_INVALID_ARG, "negative")
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 4, -16, 4, 0, FAKE, None, None),
            H.RNN_ERR_INVALID_ARG, "negative")
    _status(lib.rnn_igemm(FAKE, FAKE, FAKE, 1, 1, -1, None, 0, None), H.RNN_ERR_INVALID_ARG,
            "negative")


def test_gemm_argument_rules(lib):
    # unknown flag bits
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 4, 16, 4, 0x100, FAKE, None, None),
            H.RNN_ERR_INVALID_ARG, "unknown flags")
    # neither output requested
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 4, 16, 4, 0, None, None, None),
            H.RNN_ERR_INVALID_ARG, "both null")
    # float output needs the scales
    _status(lib.rnn_w8a8_linear(FAKE, None, FAKE, FAKE, None, 4, 16, 4, 0, FAKE, None, None),
            H.RNN_ERR_INVALID_ARG, "requires sa")
    # any k runs on the byte-assembling kernel, but the forced GEMV / LDS-DMA need k % 16 == 0
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 4, 17, 4, H.ALGO_GEMV, FAKE, None,
                                None), H.RNN_ERR_UNSUPPORTED, "k % 16 == 0")
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 40, 17, 4, H.ALGO_TILED_DMA, FAKE,
                                None, None), H.RNN_ERR_UNSUPPORTED, "k % 16 == 0")
    # GEMV forced beyond 16 rows
    _status(lib.rnn_w8a8_linear(FAKE, FAKE, FAKE, FAKE, None, 17, 16, 4, H.ALGO_GEMV, FAKE, None,
                                None), H.RNN_ERR_INVALID_ARG, "m <= 16")
    _status(lib.rnn_ternary_gemm(FAKE, FAKE, FAKE, FAKE, None, 4, 20, 4, H.ALGO_TILED_DMA, FAKE,
                                 None, None), H.RNN_ERR_UNSUPPORTED, "k % 128 == 0")
    _status(lib.rnn_ternary_gemm(FAKE, FAKE, ctypes.c_void_p(258), FAKE, None, 4, 32, 4, 0, FAKE,
                                 None, None), H.RNN_ERR_INVALID_ARG, "4-byte aligned")


def test_sgemm_argument_rules(lib):
    """rnn_sgemm (BlasBackend::sgemm): the leading-dimension rules of the
    reference's contract (src/blas.rs:93-101) and the transpose flags."""
    def call(ta=0, tb=0, m=4, n=4, k=4, alpha=1.0, lda=4, ldb=4, ldc=4, c=FAKE):
        return lib.rnn_sgemm(ta, tb, m, n, k, alpha, FAKE, lda, FAKE, ldb, 0.0, c, ldc, None)
    _status(call(m=-1), H.RNN_ERR_INVALID_ARG, "negative")
    _status(call(ta=2), H.RNN_ERR_INVALID_ARG, "transa/transb")
    _status(call(ldc=3), H.RNN_ERR_INVALID_ARG, "ldc")
    _status(call(c=None), H.RNN_ERR_INVALID_ARG, "null C")
    _status(call(k=8, lda=7), H.RNN_ERR_INVALID_ARG, "lda")           # A [m,k]: lda >= k
    _status(call(ta=1, m=8, lda=7, ldc=8), H.RNN_ERR_INVALID_ARG, "lda")  # A [k,m]: lda >= m
    _status(call(n=8, ldb=7, ldc=8), H.RNN_ERR_INVALID_ARG, "ldb")    # B [k,n]: ldb >= n
    _status(call(tb=1, k=8, lda=8, ldb=7), H.RNN_ERR_INVALID_ARG, "ldb")  # B [n,k]: ldb >= k
    # m == 0 or n == 0 is a no-op, with no pointer needed
    assert lib.rnn_sgemm(0, 0, 0, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None) == 0
    assert lib.rnn_sgemm(0, 0, 4, 0, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None) == 0


def test_empty_shapes_are_noops(lib):
    assert lib.rnn_w8a8_linear(None, None, None, None, None, 0, 16, 4, 0, None, None, None) == 0
    assert lib.rnn_quant_rows_i8(None, 0, 5, None, None, None) == 0
    assert lib.rnn_ternary_pack(None, 0, None, None) == 0
    assert lib.rnn_rotorquant_quantize(None, 0, 12, 4, None, None, None, None, None) == 0


def test_rotorquant_argument_rules(lib):
    # RotorQuant needs at least 2 bits (src/quant.rs:136)
    _status(lib.rnn_rotorquant_quantize(FAKE, 1, 12, 1, FAKE, FAKE, None, None, None),
            H.RNN_ERR_INVALID_ARG, "at least 2 bits")
    # int8 codes hold at most 8 bits
    _status(lib.rnn_rotorquant_quantize(FAKE, 1, 12, 9, FAKE, None, FAKE, FAKE, None),
            H.RNN_ERR_INVALID_ARG, "out of range")
    _status(lib.rnn_rotorquant_quantize(FAKE, 1, 0, 4, FAKE, FAKE, None, None, None),
            H.RNN_ERR_INVALID_ARG, "dim")
    # any dim (past 2688 the kernels rebuild the rotation matrices per item);
    # a dim whose group count overflows the kernels' index type is refused
    _status(lib.rnn_rotorquant_quantize(FAKE, 1, 10**10, 4, FAKE, FAKE, None, None, None),
            H.RNN_ERR_INVALID_ARG, "too large")
    _status(lib.rnn_rotorquant_dequantize(FAKE, FAKE, 1, 10**10, FAKE, FAKE, None),
            H.RNN_ERR_INVALID_ARG, "too large")
    _status(lib.rnn_ternary_quantize(FAKE, 2, 2, 7, FAKE, FAKE, None), H.RNN_ERR_INVALID_ARG,
            "bad mode")


def test_igemm_workspace_size(lib):
    assert lib.rnn_igemm_workspace_size(0, 5, 5) == 0
    # A' [m, kp] + B^T [n, kp] + colsum [n], each rounded up to 256 bytes, kp = ceil64(k)
    assert lib.rnn_igemm_workspace_size(3, 5, 7) == 256 + 512 + 256
    assert lib.rnn_igemm_workspace_size(2048, 4096, 14336) == 2048 * 4096 + 14336 * 4096 + 14336 * 4


def test_product_path_has_no_cpu_fallback():
    # the binding refuses to run without the HIP library (no silent fallback)
    import importlib
    mod = importlib.reload(H)
    saved = mod.LIB_PATH
    try:
        mod.LIB_PATH = "/nonexistent/librnn_hip.so"
        mod._lib = None
        with pytest.raises(mod.RnnError):
            mod.load()
    finally:
        mod.LIB_PATH = saved
        mod._lib = None


def test_build_rejects_kernels_demoted_to_scratch():
    """build.py parses hipcc's resource-usage remarks and refuses a kernel that
    uses scratch (private) memory: such a kernel computes correct values but
    runs one to two orders of magnitude slower."""
    import build
    ok = ("remark: gemm.hip:10:0: Function Name: _ZN3rnn4goodEv\n"
          "remark: gemm.hip:10:0:     ScratchSize [bytes/lane]: 0\n")
    bad = ok + ("remark: gemm.hip:20:0: Function Name: _ZN3rnn3badEv\n"
                "remark: gemm.hip:20:0:     VGPRs: 88\n"
                "remark: gemm.hip:20:0:     ScratchSize [bytes/lane]: 1456\n")
    assert build._scratch_kernels(ok) == []
    assert build._scratch_kernels(bad) == ["_ZN3rnn3badEv (1456 B/lane)"]


def test_success_clears_the_error_message(lib):
    # a failing call leaves its message; the next call that succeeds clears it
    _status(lib.rnn_quant_rows_i8(FAKE, -1, 4, FAKE, FAKE, None), H.RNN_ERR_INVALID_ARG, "negative")
    assert lib.rnn_quant_rows_i8(FAKE, 0, 4, FAKE, FAKE, None) == H.RNN_OK  # empty: no launch
    assert H.last_error() == ""


def test_new_elementwise_argument_rules(lib):
    _status(lib.rnn_relu(FAKE, -1, FAKE, None), H.RNN_ERR_INVALID_ARG, "negative")
    _status(lib.rnn_bias_act(FAKE, FAKE, 2, 2, 2, None), H.RNN_ERR_INVALID_ARG, "relu must be")
    _status(lib.rnn_linear_layer(FAKE, 2, 4, FAKE, 3, None, 0, None, None), H.RNN_ERR_INVALID_ARG,
            "null pointer")
    assert lib.rnn_bias_act(FAKE, None, 4, 4, 0, None) == H.RNN_OK  # nothing to do: no launch


def test_attention_workspace_alignment(lib):
    """The attention's split counts and states take 4-byte atomics: a caller
    workspace must be 16-byte aligned, as rnn_qt_linear_forward_ws requires."""
    def call(ws):
        return lib.rnn_rotorquant_kv_attention_ws(FAKE, 32, 1, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE,
                                                   4096, 128, 0.1, FAKE, ws, 1 << 20, None)
    _status(call(ctypes.c_void_p(258)), H.RNN_ERR_INVALID_ARG, "16-byte aligned")
    _status(lib.rnn_qt_linear_forward_ws(3, FAKE, 1, 4096, FAKE, 1 << 20, FAKE, 1 << 15, 128,
                                         11008, None, FAKE, ctypes.c_void_p(260), 1 << 24, 0, None),
            H.RNN_ERR_INVALID_ARG, "misaligned")


# ------------------------------------------------- binding size checks (no GPU)
class _Stand:
    """Quacks like a contiguous device tensor for the binding's argument checks;
    its pointer is never used, because every case below must fail before the
    C ABI is called (on this GPU-less host a call would not reach a kernel)."""

    def __init__(self, shape, dtype):
        self.shape, self.dtype, self.is_cuda = tuple(shape), dtype, True

    def dim(self):
        return len(self.shape)

    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def is_contiguous(self):
        return True

    def data_ptr(self):
        return 256

    def element_size(self):
        return 1


def _rejects(fn, needle):
    with pytest.raises(H.RnnError) as e:
        fn()
    assert e.value.status == H.RNN_ERR_INVALID_ARG and needle in str(e.value), str(e.value)


def test_binding_checks_buffer_sizes_before_the_call():
    import torch
    i8, f32, i32, u8 = torch.int8, torch.float32, torch.int32, torch.uint8
    aq, wq = _Stand((4, 64), i8), _Stand((8, 64), i8)
    sa, sw = _Stand((4,), f32), _Stand((8,), f32)
    _rejects(lambda: H.w8a8_linear(aq, sa, _Stand((8, 32), i8), sw), "k=32")
    _rejects(lambda: H.w8a8_linear(aq, _Stand((3,), f32), wq, sw), "sa holds 3")
    _rejects(lambda: H.w8a8_linear(aq, sa, wq, _Stand((7,), f32)), "sw holds 7")
    _rejects(lambda: H.w8a8_linear(aq, sa, wq, sw, bias=_Stand((9,), f32)), "bias holds 9")
    _rejects(lambda: H.w8a8_linear(aq, sa, wq, sw, y=_Stand((4, 7), f32)), "y holds 28")
    _rejects(lambda: H.w8a8_linear(aq, sa, wq, sw, y=_Stand((4, 8), i32)), "y must be")
    _rejects(lambda: H.igemm(_Stand((4, 63), u8), _Stand((64, 8), i8), 4, 64, 8), "a holds 252")
    _rejects(lambda: H.igemm(_Stand((4, 64), u8), _Stand((64, 8), i8), 4, 64, 8,
                             c=_Stand((4, 9), i32)), "c holds 36")
    _rejects(lambda: H.quant_rows_i8(_Stand((4, 64), f32), q=_Stand((4, 60), i8)), "q holds 240")
    _rejects(lambda: H.ternary_gemm(aq, sa, _Stand((8 * 64 // 16 - 1,), i32), sw, 8), "packed holds")
    _rejects(lambda: H.qt_linear_forward(3, _Stand((2, 64), f32), _Stand((256,), u8),
                                         _Stand((4,), f32), 32, 8, y=_Stand((2, 7), f32)), "y holds 14")
    _rejects(lambda: H.rotorquant_quantize(_Stand((5, 128), f32), _Stand((42, 4), f32), 4),
             "rotors holds 168")
    _rejects(lambda: H.rotorquant_quantize(_Stand((5, 128), f32), _Stand((43, 4), f32), 4,
                                           y=_Stand((5, 127), f32)), "y holds 635")
    # a cache page shorter than the sequence the attention is told to read
    nc, ns = 2 * 64 * 8 * 6, 2 * 64 * 4 * 11
    pages = ((_Stand((nc,), torch.int16), _Stand((ns - 4,), f32)),
             (_Stand((nc,), torch.int16), _Stand((ns,), f32)))
    _rejects(lambda: H.rotorquant_kv_attention(_Stand((2, 1, 128), f32), pages[0], pages[1],
                                               _Stand((43, 4), f32), _Stand((43, 4), f32), 64, 0.1),
             "k scales holds")
    _rejects(lambda: H.sgemm(0, 0, 4, 4, 4, 1.0, _Stand((15,), f32), 4, _Stand((16,), f32), 4, 0.0,
                             _Stand((16,), f32), 4), "a holds 15")
    _rejects(lambda: H.linear_layer(_Stand((2, 64), f32), _Stand((8, 32), f32)), "w expects 32")
