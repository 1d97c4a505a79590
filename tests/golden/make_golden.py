"""Writes tests/golden/golden_small.npz: small input/output vectors for every
function on the quantized-inference path, computed by the CPU oracle.

Test data, not product code. The reference (Rust) cannot be built or run in
this image, so the expected outputs come from the oracle after it has been
pinned by the reference's own known-answer tests, brute force and closed forms
(tests/test_oracle.py). Two things use the fixture:
  - tests/test_golden.py (CPU) recomputes every output with the oracle and
    demands bit equality, so a change to the oracle cannot pass silently;
  - tests/test_gpu_golden.py runs the HIP library on the same inputs.

Where a case mirrors a reference test, its inputs are that test's inputs and
the citation is given. Regenerate with `python tests/golden/make_golden.py`
after `make -C oracle`; the archive is written without pickles
(numpy.load(..., allow_pickle=False) reads it).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "rust-neural-network_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle as O  # noqa: E402
import workloads as W  # noqa: E402

OUT = os.path.join(HERE, "golden_small.npz")


def special_rows(rows, cols, seed):
    """Activations with the edge cases of the per-row int8 rule: an all-zero
    row, a row whose quotients x/scale land exactly on .5 (half-away rounding,
    src/int8.rs:41-42), and a row with one large outlier."""
    x = W.activations(rows, cols, seed=seed)
    x[1] = 0.0
    halves = (np.arange(cols, dtype=np.float32) % 9 - 4) + np.float32(0.5)
    halves[0] = np.float32(127.0)                        # max-abs 127 -> scale exactly 1.0
    x[2] = halves
    x[3, cols // 2] = np.float32(300.0)
    return x


def cases() -> dict[str, np.ndarray]:
    g: dict[str, np.ndarray] = {}

    # --- igemm: the reference's known answer (src/int8.rs:416-422) and an LCG case
    # built the way the reference's bench/test inputs are (src/int8.rs:382-394, 425-433).
    g["igemm_kat.a"] = np.array([[1, 2, 3, 4]], np.uint8)
    g["igemm_kat.b"] = np.array([[1, -1], [2, 2], [-3, 4], [0, -2]], np.int8)
    g["igemm_kat.c"] = O.igemm_scalar(g["igemm_kat.a"], g["igemm_kat.b"], 1, 4, 2)
    m, k, n = 16, 64, 24
    a, s = O.lcg_bytes(12345, m * k, signed=False)
    b, _ = O.lcg_bytes(s, k * n, signed=True)
    g["igemm_lcg.a"] = a.view(np.uint8).reshape(m, k)
    g["igemm_lcg.b"] = b.reshape(k, n)
    g["igemm_lcg.c"] = O.igemm_scalar(g["igemm_lcg.a"], g["igemm_lcg.b"], m, k, n)

    # --- per-row int8 quantization and dequantization (src/int8.rs:24-61)
    x = special_rows(6, 37, seed=11)
    q, sc = O.quant_rows_i8(x)
    g["quant_rows.x"], g["quant_rows.q"], g["quant_rows.scale"] = x, q, sc
    g["int8_dequant.w"] = O.int8_dequantize(q, sc)

    # --- Int8Weights::matmul_f32 (src/int8.rs:70-96) and Int8Linear::forward (:134-172)
    w = W.weights(8, 40, seed=12, std=0.5)
    wq, ws = O.quant_rows_i8(w)
    xi = W.activations(3, 40, seed=13)
    bias8 = W.rng(14).standard_normal(8).astype(np.float32)
    g["int8_lin.wq"], g["int8_lin.ws"], g["int8_lin.x"], g["int8_lin.bias"] = wq, ws, xi, bias8
    g["int8_lin.matmul_y"] = O.int8_matmul_f32(wq, ws, xi)
    g["int8_lin.forward_y"] = O.int8_linear_forward(xi, wq, ws, bias8)

    # --- W8A8 linear: int32 accumulate + per-channel dequant (+bias, ReLU)
    m, k, n = 5, 256, 24
    aq, sa = O.quant_rows_i8(special_rows(m, k, seed=15))
    wq, sw = O.quant_rows_i8(W.weights(n, k, seed=16))
    bias = W.rng(17).standard_normal(n).astype(np.float32)
    g["w8a8.aq"], g["w8a8.sa"], g["w8a8.wq"], g["w8a8.sw"], g["w8a8.bias"] = aq, sa, wq, sw, bias
    g["w8a8.y"], g["w8a8.acc"] = O.w8a8_linear(aq, sa, wq, sw, None, False)
    g["w8a8.y_bias_relu"], _ = O.w8a8_linear(aq, sa, wq, sw, bias, True)

    # --- ternary packing: the reference's round-trip vectors (src/ternary.rs:427-446)
    kat = np.array([1, -1, 0, 1, -1, 0, 1, 1, -1, -1, 0, 0, 1, -1, 1, 0], np.int8)
    g["ternary_pack_kat.t"] = kat
    g["ternary_pack_kat.packed"] = O.pack_ternary(kat)
    big = np.array([(1, -1, 0)[i % 3] for i in range(1000)], np.int8)
    g["ternary_pack_large.t"] = big
    g["ternary_pack_large.packed"] = O.pack_ternary(big)

    # --- TernaryTensor::quantize, per-row rule (src/ternary.rs:97-138), with the
    # reference's value-count matrix (src/ternary.rs:412-424) as its first two rows.
    wt = W.weights(6, 40, seed=18, std=1.0)
    wt[:2] = 0.0
    wt[0, :4] = [10.0, -10.0, 0.001, -0.001]
    wt[1, :4] = [10.0, -10.0, 10.0, -10.0]
    t, st = O.ternary_quantize_rows(wt)
    g["ternary_rows.w"], g["ternary_rows.packed"], g["ternary_rows.scale"] = wt, O.pack_ternary(t), st
    g["ternary_dequant.w"] = O.ternary_dequantize(O.pack_ternary(t), wt.size, st, wt.shape[1])

    # --- absmean rule (one gamma per tensor, the BitNet b1.58 recipe)
    wa = W.ternary_latent(24, 256, seed=19)
    ta, gamma = O.ternary_quantize_absmean(wa)
    g["ternary_absmean.w"], g["ternary_absmean.packed"] = wa, O.pack_ternary(ta)
    g["ternary_absmean.gamma"] = np.array([gamma], np.float32)

    # --- TernaryLinear::forward, f32 shift-and-add (src/ternary.rs:239-279)
    xt = W.activations(3, 40, seed=20)
    bias6 = W.rng(21).standard_normal(6).astype(np.float32)
    g["ternary_lin.x"], g["ternary_lin.bias"] = xt, bias6
    g["ternary_lin.y"] = O.ternary_linear_f32(xt, O.pack_ternary(t), st, 6, bias6)

    # --- int8 ternary GEMM on the absmean weights
    aq, sa = O.quant_rows_i8(special_rows(5, 256, seed=22))
    swt = np.full(24, gamma, np.float32)
    bias24 = W.rng(23).standard_normal(24).astype(np.float32)
    g["ternary_gemm.aq"], g["ternary_gemm.sa"], g["ternary_gemm.bias"] = aq, sa, bias24
    g["ternary_gemm.y"], g["ternary_gemm.acc"] = O.ternary_gemm_i8(
        aq, sa, g["ternary_absmean.packed"], swt, 24, None, False)
    g["ternary_gemm.y_bias_relu"], _ = O.ternary_gemm_i8(
        aq, sa, g["ternary_absmean.packed"], swt, 24, bias24, True)

    # --- Cl(3,0) rotor rotation matrices (src/quant.rs:101-120), unit, identity and non-unit
    r = W.rotors(8, seed=24)
    r[0] = (1.0, 0.0, 0.0, 0.0)
    r[1] = (2.0, 0.5, -1.0, 0.25)
    g["rotor_mats.rotors"] = r
    g["rotor_mats.m"] = np.stack([O.rotor_rotation_matrix(v) for v in r])

    # --- RotorQuant: the reference test's data and bound (src/quant.rs:291-310):
    # dim 12, 4 bits, data i*0.37-1.5, error < 0.15 x range. The reference's
    # with_seed(12, 4, 123) draws its rotors from rand's StdRng, which is not in this
    # image; the rotors here come from the build's own seeded generator (the formula
    # of Rotor::random, src/quant.rs:39-65) and are stored with the case.
    rq_r = W.rotors(4, seed=123)
    data = (np.arange(12, dtype=np.float32) * np.float32(0.37) - np.float32(1.5)).reshape(1, 12)
    y, c, s = O.rotorquant_quantize(data, rq_r, 4)
    g["rq_ref.x"], g["rq_ref.rotors"], g["rq_ref.y"], g["rq_ref.codes"], g["rq_ref.scales"] = \
        data, rq_r, y, c, s

    # --- RotorQuant at the KV head width and a ragged one, 3/4/8 bits, with a
    # zero group and a row below the 1e-12 skip threshold (src/quant.rs:189-191)
    for dim in (128, 10):
        xr = W.activations(6, dim, seed=25 + dim)
        xr[0, :3] = 0.0
        xr[1] *= np.float32(1e-13)
        rr = W.rotors((dim + 2) // 3, seed=26 + dim)
        g[f"rq_d{dim}.x"], g[f"rq_d{dim}.rotors"] = xr, rr
        for bits in (3, 4, 8):
            y, c, s = O.rotorquant_quantize(xr, rr, bits)
            g[f"rq_d{dim}.b{bits}.y"], g[f"rq_d{dim}.b{bits}.codes"] = y, c
            g[f"rq_d{dim}.b{bits}.scales"] = s
            g[f"rq_d{dim}.b{bits}.deq"] = O.rotorquant_dequantize(c, s, dim, rr)

    # --- QuantizedTensor (src/quantize.rs): every format on the reference tests'
    # inputs -- int8_roundtrip (:825-834, group 0), nvfp4_roundtrip (:862-872,
    # group 8), fp16_roundtrip (:874-887), all_formats_produce_valid_output
    # (:939-961, a 16x16 tensor, group 32) -- and the odd-group INT4 layout
    # (group 3 over 6 elements).
    ref_inputs = {
        "int8": (np.array([0.1, 0.5, -0.3, 0.8, -0.9, 0.0], np.float32), 0),
        "nvfp4": (np.array([0.0, 0.5, 1.0, -1.5, 3.0, -6.0, 2.0, -0.5], np.float32), 8),
        "fp16": (np.array([1.0, 0.5, -0.25, 100.0, -1000.0, 0.001], np.float32), 0),
        "rand": (W.activations(16, 16, seed=27).ravel(), 32),
        "odd": (np.array([7.0, -7.0, 1.0, 3.5, 7.0, -3.5], np.float32), 3),
    }
    for tag, (x, gs) in ref_inputs.items():
        g[f"qt_{tag}.x"] = x
        g[f"qt_{tag}.gs"] = np.array([gs], np.int64)
        for f in range(9):
            d, sc, grp = O.qt_quantize(f, x, gs)
            key = f"qt_{tag}.{O.QF_NAMES[f]}"
            g[f"{key}.data"], g[f"{key}.scales"] = d, sc
            g[f"{key}.group"] = np.array([grp], np.int64)
            g[f"{key}.deq"] = O.qt_dequantize(f, d, sc, grp, x.size)

    # --- QuantizedLinear::forward (src/quantize.rs:744-754), INT4 group 32, with
    # bias; y from the oracle's sgemm order and sum|x||W| + |b| for the f32 bound
    wq = (W.rng(28).standard_normal((40, 96)) * 0.02).astype(np.float32)
    xq = W.activations(3, 96, seed=29)
    bq = W.rng(30).standard_normal(40).astype(np.float32)
    d, sc, grp = O.qt_quantize(O.QF_INT4, wq, 32)
    g["qt_linear.x"], g["qt_linear.bias"], g["qt_linear.data"], g["qt_linear.scales"] = xq, bq, d, sc
    g["qt_linear.group"] = np.array([grp], np.int64)
    g["qt_linear.y"] = O.qt_linear_forward(O.QF_INT4, xq, d, sc, grp, 40, bq)
    wdq = O.qt_dequantize(O.QF_INT4, d, sc, grp, wq.size).reshape(40, 96).astype(np.float64)
    g["qt_linear.absdot"] = np.abs(xq.astype(np.float64)) @ np.abs(wdq).T + np.abs(bq)

    # --- attention over the RotorQuant KV cache: Tensor::flash_attention
    # (src/tensor.rs:618-672) over the 4-bit reconstructions of K and V,
    # 2 sequences x 70 positions, head dim 12 (4 groups), one query each
    kx = W.activations(140, 12, seed=31)
    vx = W.activations(140, 12, seed=32)
    kr, vr = W.rotors(4, seed=33), W.rotors(4, seed=34)
    _, kcodes, ksc = O.rotorquant_quantize(kx, kr, 4)
    _, vcodes, vsc = O.rotorquant_quantize(vx, vr, 4)
    kd = O.rotorquant_dequantize(kcodes, ksc, 12, kr).reshape(2, 70, 12)
    vd = O.rotorquant_dequantize(vcodes, vsc, 12, vr).reshape(2, 70, 12)
    qa = W.activations(2, 12, seed=35).reshape(2, 1, 12)
    g["kv_attn.k_codes"], g["kv_attn.k_scales"], g["kv_attn.k_rotors"] = kcodes, ksc, kr
    g["kv_attn.v_codes"], g["kv_attn.v_scales"], g["kv_attn.v_rotors"] = vcodes, vsc, vr
    g["kv_attn.q"] = qa
    g["kv_attn.out"] = O.flash_attention(qa, kd, vd, np.float32(0.25))
    # tolerance between any two evaluations within the f32 bound of the exact
    # attention: 2 x (4 ds + (skv + 8) u) 2 max|V|, ds = (dim + 16) u scale
    # max_j sum_t |q_t||K_jt| (the bound the GPU tests apply)
    u = 2.0 ** -24
    sabs = np.einsum("bid,bjd->bij", np.abs(qa).astype(np.float64), np.abs(kd).astype(np.float64))
    ds = (12 + 16) * u * 0.25 * sabs.max(axis=2)
    vmax = np.abs(vd).max(axis=(1, 2))[:, None, None]
    g["kv_attn.tol"] = 2 * (4 * ds[..., None] + (70 + 8) * u) * vmax * 2
    return g


def main() -> None:
    g = cases()
    np.savez_compressed(OUT, **g)
    size = os.path.getsize(OUT)
    print(f"wrote {OUT}: {len(g)} arrays, {size} bytes")


if __name__ == "__main__":
    main()
