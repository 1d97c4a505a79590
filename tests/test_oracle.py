"""Pins the CPU oracle (oracle/liboracle.so) without the reference's toolchain.

Each test checks an oracle function against a reference known-answer test, a
brute force computed by a different method (numpy int64/float64), a closed
form, or an invariant chosen so that a dropped term, wrong sign, wrong index or
transposed operand fails. Citations are to gugu8intel-i9/Rust-Neural-Network.
"""
import itertools

import numpy as np
import pytest

import oracle as O
import workloads as W

LCG_SHAPES = [(16, 32, 48), (3, 5, 7), (13, 17, 29), (1, 1, 1), (4, 4, 16), (33, 9, 33),
              (64, 64, 64)]  # src/int8.rs:425-433


def lcg_case(m, k, n):
    """src/int8.rs:396-400: seed 1, A unsigned (masked 0x7f), then B signed."""
    a, s = O.lcg_bytes(1, m * k, signed=False)
    b, _ = O.lcg_bytes(s, k * n, signed=True)
    return a.view(np.uint8).reshape(m, k), b.reshape(k, n)


def lcg_python(seed, n, signed):
    out = []
    for _ in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xFFFFFFFF
        b = (seed >> 16) & 0xFF
        out.append(b - 256 if signed and b >= 128 else (b if signed else b & 0x7F))
    return np.array(out, np.int64), seed


# ------------------------------------------------------------------ igemm
def test_lcg_generator_matches_reference_recurrence():
    got, s = O.lcg_bytes(1, 1000, signed=True)
    exp, s2 = lcg_python(1, 1000, True)
    assert np.array_equal(got.astype(np.int64), exp) and s == s2
    got, _ = O.lcg_bytes(7, 100, signed=False)
    assert got.max() <= 127 and got.min() >= 0


@pytest.mark.parametrize("fn", ["igemm", "igemm_scalar"])
def test_igemm_known_small(fn):
    # src/int8.rs:416-422
    a = np.array([1, 2, 3, 4], np.uint8)
    b = np.array([1, -1, 2, 2, -3, 4, 0, -2], np.int8)
    c = O.igemm(a, b, 1, 4, 2)[0] if fn == "igemm" else O.igemm_scalar(a, b, 1, 4, 2)
    assert c.ravel().tolist() == [-4, 7]


@pytest.mark.parametrize("shape", LCG_SHAPES)
def test_igemm_lcg_shapes_brute_force(shape):
    m, k, n = shape
    a, b = lcg_case(m, k, n)
    ref = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    assert np.array_equal(O.igemm_scalar(a, b, m, k, n), ref)
    for threads in (1, 3):
        c, _ = O.igemm(a, b, m, k, n, threads)
        assert np.array_equal(c, ref)


def test_igemm_bench_inputs_and_full_u8_range():
    # benches/core_ops.rs:152-153 inputs, 128^3 (full u8 range in A)
    n = 128
    a = (np.arange(n * n) % 251).astype(np.uint8).reshape(n, n)
    b = (np.arange(n * n) % 255).astype(np.uint8).view(np.int8).reshape(n, n)
    ref = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.int32)
    assert np.array_equal(O.igemm(a, b, n, n, n, 4)[0], ref)


def test_igemm_wraps_like_release_rust():
    # 255*127*K overflows int32 for K > 66313: wrapping arithmetic mod 2^32
    m, k, n = 1, 70000, 2
    a = np.full((m, k), 255, np.uint8)
    b = np.full((k, n), 127, np.int8)
    exp = np.int64(255 * 127 * k)
    wrapped = ((exp + 2**31) % 2**32) - 2**31
    assert np.all(O.igemm_scalar(a, b, m, k, n) == wrapped)
    assert np.all(O.igemm(a, b, m, k, n, 2)[0] == wrapped)


# ------------------------------------------------------------------ int8 quant
def test_int8_roundtrip_low_error():
    # src/int8.rs:322-327
    w = np.array([[0.1, 0.2, 0.3, -0.4], [0.5, -0.6, 0.7, 0.8]], np.float32)
    q, s = O.quant_rows_i8(w)
    deq = O.int8_dequantize(q, s)
    assert np.abs(deq - w).mean() < 0.01


def test_quant_rows_closed_form_properties():
    x = W.activations(64, 300, seed=3, outlier_frac=0.01)
    x[5] = 0.0                                  # all-zero row -> scale 1.0
    x[7, :3] = [1e30, -1e30, 5.0]               # extreme magnitudes
    q, s = O.quant_rows_i8(x)
    absmax = np.abs(x.astype(np.float64)).max(axis=1)
    assert s[5] == np.float32(1.0) and np.all(q[5] == 0)
    nz = absmax > 0
    assert np.array_equal(s[nz], (absmax[nz].astype(np.float32) / np.float32(127.0)))
    # the max-|x| element maps to +-127 exactly, every code is within +-127
    for r in np.nonzero(nz)[0]:
        j = np.argmax(np.abs(x[r]))
        assert abs(int(q[r, j])) == 127
    assert q.min() >= -127 and q.max() <= 127
    # reconstruction within half a step (independent float64 check)
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert np.all(err <= s[:, None].astype(np.float64) * (0.5 + 1e-5))


def test_quant_rows_rounds_half_away_from_zero():
    # scale = 127/127 = 1: ratios are the values themselves
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]], np.float32)
    q, s = O.quant_rows_i8(x)
    assert s[0] == 1.0
    assert q[0].tolist() == [127, 3, -3, 1, -1, 2, -127, 3]


def test_quant_rows_nan_maps_to_zero():
    x = np.array([[np.nan, 1.0, -2.0]], np.float32)
    q, s = O.quant_rows_i8(x)
    assert s[0] == np.float32(2.0) / np.float32(127.0)  # f32::max ignores NaN
    assert q[0].tolist() == [0, 64, -127]


def test_int8_linear_forward_exact_when_ratios_are_integers():
    # src/int8.rs:134-172 with s[o] = 0.5 and x multiples of 0.5: a_q = 2x exactly
    rng = W.rng(11)
    batch, in_f, out_f = 3, 20, 6
    x = (rng.integers(-40, 41, (batch, in_f)) * 0.5).astype(np.float32)
    wq = rng.integers(-128, 128, (out_f, in_f)).astype(np.int8)
    ws = np.full(out_f, 0.5, np.float32)
    bias = rng.standard_normal(out_f).astype(np.float32)
    acc = (2 * x).astype(np.int64) @ wq.astype(np.int64).T
    exp = (acc.astype(np.float32) * ws * ws + bias).astype(np.float32)
    assert np.array_equal(O.int8_linear_forward(x, wq, ws, bias), exp)
    # saturation: |x/s| > 127 clamps to 127 / -128
    xs = np.full((1, in_f), 1000.0, np.float32)
    xs[0, ::2] = -1000.0
    acc_s = np.where(np.arange(in_f) % 2 == 0, -128, 127).astype(np.int64) @ wq.astype(np.int64).T
    exp_s = (acc_s.astype(np.float32) * ws * ws).astype(np.float32)
    assert np.array_equal(O.int8_linear_forward(xs, wq, ws), exp_s[None, :])


def test_int8_linear_matches_f32_approximately():
    # src/int8.rs:346-369 (Linear::new(8, 4): He init, x ~ N(0,1)), max diff < 5
    rng = W.rng(5)
    w = (rng.standard_normal((4, 8)) * np.sqrt(2.0 / 8)).astype(np.float32)
    x = rng.standard_normal((2, 8)).astype(np.float32)
    wq, ws = O.quant_rows_i8(w)
    y = O.int8_linear_forward(x, wq, ws, np.zeros(4, np.float32))
    assert np.abs(y - x @ w.T).max() < 5.0


def test_int8_matmul_f32_uses_reciprocal():
    # src/int8.rs:79: x * (1.0/scale), not x / scale. With scale 0.3 and
    # x = -17.25: x * fl(1/0.3) = -57.5 -> -58, while x / 0.3 = -57.499996 -> -57.
    wq = np.ones((1, 1), np.int8)
    s = np.float32(0.3)
    ws = np.array([s], np.float32)
    x = np.array([[-17.25]], np.float32)
    assert np.float32(-17.25) * (np.float32(1.0) / s) == np.float32(-57.5)
    assert np.float32(-17.25) / s > np.float32(-57.5)
    assert O.int8_matmul_f32(wq, ws, x)[0, 0] == np.float32(-58.0) * s * s
    assert O.int8_linear_forward(x, wq, ws)[0, 0] == np.float32(-57.0) * s * s


def test_w8a8_linear_brute_force():
    m, k, n = 9, 96, 33
    rng = W.rng(21)
    aq = rng.integers(-128, 128, (m, k)).astype(np.int8)
    wq = rng.integers(-128, 128, (n, k)).astype(np.int8)
    sa = rng.random(m).astype(np.float32) + np.float32(0.01)
    sw = rng.random(n).astype(np.float32) * np.float32(0.01)
    bias = rng.standard_normal(n).astype(np.float32)
    acc_ref = (aq.astype(np.int64) @ wq.astype(np.int64).T).astype(np.int32)
    for relu in (False, True):
        y, acc = O.w8a8_linear(aq, sa, wq, sw, bias, relu)
        assert np.array_equal(acc, acc_ref)
        exp = (acc_ref.astype(np.float32) * sa[:, None]) * sw[None, :] + bias[None, :]
        if relu:
            exp = np.maximum(exp, np.float32(0.0))
        assert np.array_equal(y, exp.astype(np.float32))


def test_relu_matches_f32_max():
    x = np.array([-1.0, 0.0, 2.5, -0.0, np.nan], np.float32)
    assert O.relu(x).tolist() == [0.0, 0.0, 2.5, 0.0, 0.0]


# ------------------------------------------------------------------ ternary
def test_ternary_pack_known_word():
    # src/ternary.rs:427-432 values; codes from the table at src/ternary.rs:9-14
    v = np.array([1, -1, 0, 1, -1, 0, 1, 1, -1, -1, 0, 0, 1, -1, 1, 0], np.int8)
    p = O.pack_ternary(v)
    assert p.tolist() == [0x190A5249]
    assert np.array_equal(O.unpack_ternary(p, 16), v)


def test_ternary_pack_unpack_large():
    # src/ternary.rs:435-446
    v = np.array([(1, -1, 0)[i % 3] for i in range(1000)], np.int8)
    p = O.pack_ternary(v)
    assert p.size == 63
    assert np.array_equal(O.unpack_ternary(p, 1000), v)


def test_ternary_unpack_code_11_is_zero_and_pack_saturates():
    assert O.unpack_ternary(np.array([0xFFFFFFFF], np.uint32), 16).tolist() == [0] * 16
    # pack: any v > 0 -> 01, v < 0 -> 10 (src/ternary.rs:54-55)
    assert O.pack_ternary(np.array([5, -7, 0, 127], np.int8)).tolist() == [0b01_00_10_01]


def test_ternary_value_counts_reference_rule():
    # src/ternary.rs:412-424: row0 mean 5.0005 -> threshold 3.50035 -> [1,-1,0,0]
    w = np.array([[10.0, -10.0, 0.001, -0.001], [10.0, -10.0, 10.0, -10.0]], np.float32)
    t, s = O.ternary_quantize_rows(w)
    assert t.tolist() == [[1, -1, 0, 0], [1, -1, 1, -1]]
    assert s[1] == np.float32(10.0)
    # src/ternary.rs:401-410: small values become 0
    t2, _ = O.ternary_quantize_rows(np.array([[0.5, -0.5, 0.01, -0.01]] * 2, np.float32))
    assert (t2 == 0).sum() == 4


def test_ternary_rows_sequential_sum_and_floor_scale():
    w = np.zeros((2, 5), np.float32)
    w[1] = [1e-12, 0, 0, 0, 0]
    t, s = O.ternary_quantize_rows(w)
    assert s.tolist() == [np.float32(1e-8), np.float32(1e-8)]  # max(mean, 1e-8)
    assert t[1].tolist() == [1, 0, 0, 0, 0]  # |w| >= 0.7*mean
    # f32 sequential sum: 2^24 + 1 + 1 + ... stays 2^24 (order matters)
    row = np.array([[2.0**24] + [1.0] * 7], np.float32)
    _, s2 = O.ternary_quantize_rows(row)
    assert s2[0] == np.float32(2.0**24) / np.float32(8.0)


def test_ternary_absmean_rule():
    w = W.ternary_latent(256, 4096, seed=4)
    t, gamma = O.ternary_quantize_absmean(w)
    assert abs(float(gamma) / float(np.abs(w.astype(np.float64)).mean()) - 1) < 1e-6
    zero_frac = (t == 0).mean()
    assert 0.30 < zero_frac < 0.32   # P(|z| < 0.5*sqrt(2/pi)) = 0.3101
    assert set(np.unique(t).tolist()) == {-1, 0, 1}
    exp = np.clip(np.sign(w) * np.floor(np.abs(w / gamma) + 0.5), -1, 1)
    assert np.array_equal(t, exp.astype(np.int8))


def test_ternary_linear_f32_exact_on_integers():
    # src/ternary.rs:239-279: integer-valued x keeps the f32 sum exact
    rng = W.rng(8)
    batch, in_f, out_f = 4, 37, 9
    t = rng.integers(-1, 2, (out_f, in_f)).astype(np.int8)
    p = O.pack_ternary(t)
    x = rng.integers(-50, 51, (batch, in_f)).astype(np.float32)
    sc = rng.random(out_f).astype(np.float32)
    bias = rng.standard_normal(out_f).astype(np.float32)
    acc = (x.astype(np.int64) @ t.astype(np.int64).T).astype(np.float32)
    exp = (acc * sc[None, :] + bias[None, :]).astype(np.float32)
    assert np.array_equal(O.ternary_linear_f32(x, p, sc, out_f, bias), exp)


def test_ternary_dequantize_and_gemm():
    rng = W.rng(9)
    n, k, m = 7, 48, 5
    t = rng.integers(-1, 2, (n, k)).astype(np.int8)
    p = O.pack_ternary(t)
    sc = rng.random(n).astype(np.float32)
    w = O.ternary_dequantize(p, n * k, sc, k).reshape(n, k)
    assert np.array_equal(w, (t.astype(np.float32) * sc[:, None]).astype(np.float32))
    aq = rng.integers(-128, 128, (m, k)).astype(np.int8)
    sa = rng.random(m).astype(np.float32)
    y, acc = O.ternary_gemm_i8(aq, sa, p, sc, n)
    assert np.array_equal(acc, (aq.astype(np.int64) @ t.astype(np.int64).T).astype(np.int32))
    assert np.array_equal(y, (acc.astype(np.float32) * sa[:, None]) * sc[None, :])


# ------------------------------------------------------------------ rotors
# Generic Cl(3,0) geometric product on basis blades (bitmask e1=1,e2=2,e3=4),
# signs from counting transpositions -- independent of the sparse 28-term
# table the reference hard-codes.
_BLADES = [0, 1, 2, 4, 3, 5, 6, 7]  # [1,e1,e2,e3,e12,e13,e23,e123]


def _blade_sign(a, b):
    a >>= 1
    s = 0
    while a:
        s += bin(a & b).count("1")
        a >>= 1
    return -1.0 if s & 1 else 1.0


def ga_product(x, y):
    out = np.zeros(8)
    for i, bi in enumerate(_BLADES):
        for j, bj in enumerate(_BLADES):
            out[_BLADES.index(bi ^ bj)] += _blade_sign(bi, bj) * x[i] * y[j]
    return out


def test_rotor_is_norm_preserving():
    # src/quant.rs:258-274 (orthogonality over 100 rotors)
    for r in W.rotors(100, seed=42):
        rot = O.rotor_rotation_matrix(r).astype(np.float64)
        assert np.abs(rot @ rot.T - np.eye(3)).max() < 1e-4


def test_rotor_sandwich_is_left_product_twice():
    """apply() of src/quant.rs:70-81 is the left product R*x except for the
    sign of its e123 row; sandwich() applies it with R then with ~R, giving
    ~R*(R*x) = |R|^2 x. So the 'rotation' is the identity scaled by |R|^2 =
    s^2+p12^2+p13^2+p23^2 -- pinned here against the generic product."""
    rng = W.rng(17)
    for r in W.rotors(50, seed=7):
        R = np.array([r[0], 0, 0, 0, r[1], r[2], r[3], 0], np.float64)
        Rrev = R * np.array([1, 1, 1, 1, -1, -1, -1, 1])
        x = np.zeros(8)
        x[1:4] = rng.standard_normal(3)
        y = O.rotor_sandwich(r, x.astype(np.float32)).astype(np.float64)
        ga = ga_product(Rrev, ga_product(R, x))
        assert np.abs(y[1:4] - ga[1:4]).max() < 1e-5
        rot = O.rotor_rotation_matrix(r).astype(np.float64)
        assert np.abs(rot - np.dot(r.astype(np.float64), r) * np.eye(3)).max() < 1e-6
        # inverse sandwich undoes the sandwich (src/quant.rs:276-289)
        xr = O.rotor_sandwich(r, O.rotor_sandwich(r, x.astype(np.float32)), inverse=True)
        assert np.abs(xr - x).max() < 1e-5


def test_rotor_non_unit_scales_by_norm_squared():
    # a non-unit rotor exposes a dropped or mis-signed term: rot = |R|^2 I
    for r in ([2.0, 0.5, -1.0, 0.25], [0.0, 1.0, 1.0, 1.0], [1.0, 0.0, 0.0, 0.0]):
        r = np.array(r, np.float32)
        rot = O.rotor_rotation_matrix(r).astype(np.float64)
        assert np.abs(rot - float(np.dot(r.astype(np.float64), r)) * np.eye(3)).max() < 1e-5


# ------------------------------------------------------------------ RotorQuant
def _rq_case(rows, dim, seed):
    x = W.activations(rows, dim, seed)
    rot = W.rotors((dim + 2) // 3, seed + 1)
    return x, rot


def test_rotorquant_round_trips_with_bounded_error():
    # src/quant.rs:291-310: dim 12, 4 bits, data i*0.37-1.5, error < 0.15*range. The
    # reference draws its rotors from rand's StdRng (with_seed(12, 4, 123)); rotors are
    # an input here (RotorQuant::rotors is a pub field), drawn by the build's own
    # seeded generator with the formula of Rotor::random (src/quant.rs:39-65).
    dim = 12
    data = (np.arange(dim, dtype=np.float32) * np.float32(0.37) - np.float32(1.5))[None, :]
    y, _, _ = O.rotorquant_quantize(data, W.rotors(4, seed=123), 4)
    rng_ = data.max() - data.min()
    assert np.abs(y - data).max() < 0.15 * rng_


@pytest.mark.parametrize("dim,bits", [(128, 4), (12, 4), (10, 3), (6, 4), (1, 2), (130, 8)])
def test_rotorquant_codes_and_error_bound(dim, bits):
    x, rot = _rq_case(40, dim, seed=dim + bits)
    y, codes, scales = O.rotorquant_quantize(x, rot, bits)
    qmax = 2 ** (bits - 1) - 1
    ng = (dim + 2) // 3
    assert codes.shape == (40, 3 * ng) and scales.shape == (40, ng)
    assert np.abs(codes).max() <= qmax
    # the largest rotated coordinate of each group maps to exactly +-qmax
    assert np.all(np.abs(codes.reshape(40, ng, 3)).max(axis=2) == qmax)
    # per group: |x - y| <= |R| * |rv - rv_hat| <= sqrt(3) * scale / 2 (+ rounding)
    xp = np.zeros((40, 3 * ng), np.float64)
    xp[:, :dim] = x
    yp = np.zeros_like(xp)
    yp[:, :dim] = y
    d = np.linalg.norm((xp - yp).reshape(40, ng, 3), axis=2)
    # the pad lane's reconstruction is dropped, so measure real lanes only
    assert np.all(d <= np.sqrt(3) * scales * 0.5 * (1 + 1e-4) + 1e-6)
    # reconstruction from codes equals the fused round trip
    yd = O.rotorquant_dequantize(codes, scales, dim, rot)
    assert np.array_equal(yd, y)


def test_rotorquant_identity_rotor_is_plain_group_quantization():
    dim, bits = 9, 4
    x = W.activations(8, dim, seed=2)
    rot = np.tile(np.array([1, 0, 0, 0], np.float32), (3, 1))
    y, codes, scales = O.rotorquant_quantize(x, rot, bits)
    g = x.reshape(8, 3, 3)
    s = (np.abs(g).max(axis=2) / np.float32(7.0)).astype(np.float32)
    assert np.array_equal(scales, s)
    r = g / s[:, :, None]
    q = np.clip(np.sign(r) * np.floor(np.abs(r) + 0.5), -7, 7)
    assert np.array_equal(codes.reshape(8, 3, 3), q.astype(np.int8))
    assert np.array_equal(y, (q * s[:, :, None]).astype(np.float32).reshape(8, dim))


def test_rotorquant_zero_group_left_untouched():
    # src/quant.rs:189-191: max_abs < 1e-12 -> group skipped
    dim = 6
    x = np.zeros((2, dim), np.float32)
    x[0, :3] = [1e-13, -2e-13, 0.0]
    x[1, 3:] = [1.0, 2.0, -3.0]
    rot = W.rotors(2, seed=1)
    y, codes, scales = O.rotorquant_quantize(x, rot, 4)
    assert np.array_equal(y[0, :3], x[0, :3])
    assert scales[0, 0] == 0.0 and np.all(codes[0, :3] == 0)
    assert scales[1, 0] == 0.0 and scales[1, 1] > 0


# ------------------------------------------------------------------ f32 GEMM
def _sgemm_bound(k, scale):
    # |computed - exact| <= gamma_(k+2) * (|alpha| |A||B| + |beta C|), gamma_j = j u / (1 - j u)
    u = 2.0 ** -24
    return (k + 2) * u / (1 - (k + 2) * u) * scale + 1e-30


def test_blas_rand_mat_matches_reference_recurrence():
    # s = 1: first draws of the reference's rand_mat (src/blas.rs tests)
    v, s = O.blas_rand_mat(1, 3)
    seq, t = [], 1
    for _ in range(3):
        t = (t * 1664525 + 1013904223) % 2 ** 32
        seq.append((t >> 8) / 2 ** 24 - 0.5)
    assert np.array_equal(v, np.array(seq, np.float32)) and s == t


@pytest.mark.parametrize("case", O.BLAS_TEST_CASES, ids=[c[0] for c in O.BLAS_TEST_CASES])
def test_sgemm_reference_cases(case):
    """The reference's sgemm tests (src/blas.rs:1195-1470): same generator,
    shapes, strides, alpha/beta; within the reference's tolerance and within
    the k-term rounding bound of the float64 product."""
    _, ta, tb, m, n, k, seed, alpha, beta, tol = case
    a, lda, b, ldb, c0 = O.blas_test_case(ta, tb, m, n, k, seed, beta)
    c = O.sgemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, n).reshape(m, n)
    exact, scale = O.sgemm_f64(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c0, n)
    err = np.abs(c - exact)
    assert err.max() < tol
    assert np.all(err <= _sgemm_bound(k, scale))


def test_sgemm_known_answers_and_edges():
    # matmul_convenience_works (src/blas.rs:1514-1520)
    c = O.sgemm(0, 0, 2, 2, 2, 1.0, [1, 2, 3, 4], 2, [5, 6, 7, 8], 2, 0.0, np.zeros(4), 2)
    assert c.tolist() == [19.0, 22.0, 43.0, 50.0]
    # sgemm_zero_and_small_edges (:1471-1512): k = 0 with beta = 0 zeroes C; 1x1
    assert O.sgemm(0, 0, 2, 2, 0, 1.0, [0], 0, [0], 0, 0.0, np.full(4, 7.0), 2).tolist() == [0.0] * 4
    assert O.sgemm(0, 0, 1, 1, 1, 1.0, [3.0], 1, [4.0], 1, 0.0, [0.0], 1).tolist() == [12.0]
    # beta = 0 overwrites NaN; alpha = 0 gives beta*C; beta = 1 keeps C
    nanc = np.full(4, np.nan, np.float32)
    assert O.sgemm(0, 0, 2, 2, 1, 1.0, [1, 1], 1, [1, 1], 2, 0.0, nanc, 2).tolist() == [1.0] * 4
    assert O.sgemm(0, 0, 2, 2, 3, 0.0, np.ones(6), 3, np.ones(6), 2, 2.0,
                   np.arange(4.0), 2).tolist() == [0.0, 2.0, 4.0, 6.0]
    # leading dimensions beyond the logical sizes: padding is read as nothing
    # and left untouched in C
    a = np.array([1, 2, 99, 3, 4, 99], np.float32)           # [2,2], lda 3
    c = O.sgemm(0, 0, 2, 2, 2, 1.0, a, 3, [5, 6, 7, 8], 2, 0.0, np.full(6, -1.0), 3)
    assert c.tolist() == [19.0, 22.0, -1.0, 43.0, 50.0, -1.0]
