"""CPU pins of the oracle's QuantizedTensor restatement (src/quantize.rs).

What pins each part, without running the reference:
- the reference's own tests (src/quantize.rs:824-992): error bounds, the
  NVFP4 and f16 special values, compression ratios, finite outputs;
- f16_to_f32: every one of the 65,536 half patterns against numpy's exact
  float16 -> float32 widening;
- f32_to_f16 (truncating): the round trip over every non-NaN half and the
  toward-zero characterisation |h| <= |x| < |next half up| on random floats,
  subnormals and the overflow edge;
- f32_to_bf16: finite values against torch's round-to-nearest-even, and the
  NaN/wrap-around cases that follow from its integer formula;
- codes and scales: an independent numpy vectorisation (float32 division,
  half-away rounding evaluated in float64, argmin with first-minimum ties) on
  random data with planted ties and zero groups;
- hand-computed known answers for the odd-group 4-bit layout (each group
  packed on its own, dequantized through data[i/2]) and for Q4_0's negative
  scale (max/-8), which saturates the largest negative value at -7.
"""
import numpy as np
import pytest

import oracle as O

ALL = [O.QF_FP16, O.QF_BF16, O.QF_INT8, O.QF_INT4, O.QF_NF4, O.QF_NVFP4, O.QF_GGUF_Q4,
       O.QF_GGUF_Q4K, O.QF_GGUF_Q8]
NF4 = np.array([-1.0, -0.6961928, -0.52507305, -0.3949175, -0.28444138, -0.18477343,
                -0.091050036, 0.0, 0.0795803, 0.1609302, 0.2461123, 0.33791524, 0.44070983,
                0.562617, 0.72295684, 1.0], np.float32)
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)


def err(fmt, x, gs):
    d, s, g = O.qt_quantize(fmt, x, gs)
    dq = O.qt_dequantize(fmt, d, s, g, x.size)
    return float(np.abs(dq - x.ravel()).sum() / max(x.size, 1)), d, s


def ratio(x, d, s):
    return x.size * 4 / (d.size + s.size * 4)


# ----------------------------------------------------- the reference's own tests
def test_ref_int8_roundtrip():
    x = np.array([0.1, 0.5, -0.3, 0.8, -0.9, 0.0], np.float32)
    d, s, g = O.qt_quantize(O.QF_INT8, x, 0)
    assert g == 6 and s.size == 1
    assert np.all(np.abs(O.qt_dequantize(O.QF_INT8, d, s, g, 6) - x) < 0.05)


def test_ref_int4_compression():
    x = np.random.default_rng(1).standard_normal((64, 128)).astype(np.float32)
    _, d, s = err(O.QF_INT4, x, 32)
    assert ratio(x, d, s) > 5.0


def test_ref_nf4_lower_error_than_int4():
    x = np.random.default_rng(2).standard_normal(256).astype(np.float32)
    assert err(O.QF_NF4, x, 64)[0] <= err(O.QF_INT4, x, 64)[0] * 1.5


def test_ref_nvfp4_roundtrip():
    x = np.array([0.0, 0.5, 1.0, -1.5, 3.0, -6.0, 2.0, -0.5], np.float32)
    d, s, g = O.qt_quantize(O.QF_NVFP4, x, 8)
    dq = O.qt_dequantize(O.QF_NVFP4, d, s, g, 8)
    assert abs(dq[0]) < 0.01 and abs(dq[5] + 6.0) < 0.1
    # every value is an E2M1 point times scale 1, so the round trip is exact
    assert s[0] == 1.0 and np.array_equal(dq, x)


def test_ref_fp16_bf16_roundtrip():
    x = np.array([1.0, 0.5, -0.25, 100.0, -1000.0, 0.001], np.float32)
    d, _, _ = O.qt_quantize(O.QF_FP16, x, 0)
    dq = O.qt_dequantize(O.QF_FP16, d, np.zeros(0, np.float32), 0, x.size)
    assert np.all(np.abs(x - dq) / np.maximum(np.abs(x), 1e-6) < 0.01)
    x = np.array([1.0, -2.5, 100.0, -1000.0], np.float32)
    d, _, _ = O.qt_quantize(O.QF_BF16, x, 0)
    assert np.all(np.abs(O.qt_dequantize(O.QF_BF16, d, np.zeros(0, np.float32), 0, 4) - x) < 1.0)


def test_ref_gguf_errors():
    rng = np.random.default_rng(3)
    assert err(O.QF_GGUF_Q4, rng.standard_normal(32).astype(np.float32), 32)[0] < 0.5
    assert err(O.QF_GGUF_Q8, rng.standard_normal(64).astype(np.float32), 32)[0] < 0.05


def test_ref_all_formats_finite_and_bits():
    x = np.random.default_rng(4).standard_normal((16, 16)).astype(np.float32)
    for f in ALL:
        d, s, g = O.qt_quantize(f, x, 32)
        assert np.all(np.isfinite(O.qt_dequantize(f, d, s, g, 256)))
    assert O.QF_BITS[O.QF_FP16] == 16 and O.QF_BITS[O.QF_INT8] == 8
    assert O.QF_BITS[O.QF_NF4] == 4 and O.QF_BITS[O.QF_NVFP4] == 4
    assert abs(32 / O.QF_BITS[O.QF_INT4] - 8.0) < 0.1


def test_ref_f16_special_values_and_group_size():
    assert O.lib().orc_f32_to_f16(0.0) == 0 and O.lib().orc_f16_to_f32(0) == 0.0
    assert abs(O.lib().orc_f16_to_f32(O.lib().orc_f32_to_f16(1.0)) - 1.0) < 0.01
    assert O.lib().orc_f32_to_f16(float("inf")) & 0x7C00 == 0x7C00
    x = np.random.default_rng(5).standard_normal(256).astype(np.float32)
    assert err(O.QF_INT4, x, 32)[0] <= err(O.QF_INT4, x, 256)[0]


# ----------------------------------------------------- half / bfloat conversions
def test_f16_to_f32_exhaustive_vs_numpy():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f32_to_f16_roundtrip_and_truncation():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16)
    keep = ~np.isnan(f)
    back = O.f32_to_f16(f[keep].astype(np.float32))
    assert np.array_equal(back, h[keep])
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.uniform(-9, 5, 3000),
                        np.array([65503.9, 65504.0, 65519.99, 65520.0, 65535.9, 65536.0,
                                  6.1e-5, 5.96e-8, 2.9e-8, 1e-12])]).astype(np.float32)
    x = np.concatenate([x, -x])
    hx = O.f32_to_f16(x)
    mag = np.abs(hx.view(np.float16).astype(np.float64))
    ax = np.abs(x.astype(np.float64))
    fin = ax < 65536.0
    assert np.all(mag[fin] <= ax[fin])                     # toward zero
    nxt = (hx & 0x7FFF) + 1                                # next half up in magnitude
    up = nxt.astype(np.uint16).view(np.float16).astype(np.float64)
    assert np.all(ax[fin] < up[fin])
    assert np.all(hx[~fin] & 0x7FFF == 0x7C00)             # overflow -> Inf
    assert np.array_equal(np.signbit(hx.view(np.float16)), np.signbit(x))
    assert O.lib().orc_f32_to_f16(float("nan")) == 0x7E00


def test_bf16_vs_torch_rne_and_quirks():
    import torch
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-30, 30, 20000)).astype(np.float32)
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -3.4e38,
                                     1e-40, 0.0, -0.0], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), want)
    assert np.array_equal(O.bf16_to_f32(want).view(np.uint32), want.astype(np.uint32) << 16)
    # the integer formula on NaN payloads: 0x7F800001 + 0x7FFF -> 0x7F80 (Inf),
    # 0xFFFFFFFF + 1 + 0x7FFF wraps to 0x00007FFF -> 0x0000
    nan = np.array([0x7FC00000, 0x7F800001, 0xFFFFFFFF], np.uint32).view(np.float32)
    assert list(O.f32_to_bf16(nan)) == [0x7FC0, 0x7F80, 0x0000]


# ----------------------------------------------------- codes: independent numpy
def round_away(t32):
    t = t32.astype(np.float64)
    return np.where(t >= 0, np.floor(t + 0.5), -np.floor(-t + 0.5))


def np_quantize(fmt, x, gs):
    n = x.size
    g = n if gs == 0 else gs
    if fmt in (O.QF_GGUF_Q4, O.QF_GGUF_Q4K, O.QF_GGUF_Q8):
        g = min(g, 32)
    data, scales = [], []
    for start in range(0, n, g):
        grp = x[start:start + g]
        m = np.float32(np.max(np.abs(grp), initial=0.0))
        if fmt in (O.QF_INT8, O.QF_GGUF_Q8):
            s = m / np.float32(127) if m > 0 else np.float32(1)
        elif fmt == O.QF_INT4:
            s = m / np.float32(7) if m > 0 else np.float32(1)
        elif fmt == O.QF_NF4:
            s = m if m > 0 else np.float32(1)
        elif fmt == O.QF_NVFP4:
            s = m / np.float32(6) if m > 0 else np.float32(1)
        else:
            s = m / np.float32(-8)
            s = np.float32(1) if s == 0 else s
        scales.append(np.float32(s))
        t = (grp / np.float32(s)).astype(np.float32)
        if fmt in (O.QF_INT8, O.QF_GGUF_Q8):
            data.append(np.clip(round_away(t), -128, 127).astype(np.int8).view(np.uint8))
            continue
        if fmt in (O.QF_INT4, O.QF_GGUF_Q4, O.QF_GGUF_Q4K):
            c = (np.clip(round_away(t), -8, 7).astype(np.int64) & 0xF).astype(np.uint8)
        elif fmt == O.QF_NF4:
            c = np.argmin(np.abs(NF4[None, :] - t[:, None]), axis=1).astype(np.uint8)
        else:
            c = np.argmin(np.abs(E2M1[None, :] - np.abs(t)[:, None]), axis=1).astype(np.uint8)
            c |= np.where(t < 0, 8, 0).astype(np.uint8)
        if c.size % 2:
            c = np.append(c, np.uint8(0))
        data.append(c[0::2] | (c[1::2] << 4))
    return np.concatenate(data) if data else np.zeros(0, np.uint8), np.array(scales, np.float32)


@pytest.mark.parametrize("fmt", [f for f in ALL if f not in (O.QF_FP16, O.QF_BF16)])
@pytest.mark.parametrize("n,gs", [(1000, 32), (999, 33), (4096, 128), (77, 0), (64, 7)])
def test_codes_vs_numpy(fmt, n, gs):
    rng = np.random.default_rng(n * 31 + gs)
    x = rng.standard_normal(n).astype(np.float32) * 0.05
    x[: min(n, 2 * max(gs, 1))] = 0.0                        # zero groups (scale 1)
    if n > 200:                                              # planted exact ties: x = (k+0.5)*s
        x[150] = np.float32(0.35)
        x[151] = np.float32(-0.35)
    d, s, _ = O.qt_quantize(fmt, x, gs)
    dn, sn = np_quantize(fmt, x, gs)
    assert np.array_equal(s.view(np.uint32), sn.view(np.uint32))
    assert np.array_equal(d, dn)


def test_nf4_nvfp4_nearest_on_grid():
    """Every NF4 / E2M1 grid point maps to its own code, and midpoints break
    toward the first (lower-index) neighbour."""
    x = np.concatenate([NF4, [1.0]]).astype(np.float32)       # max 1 -> scale 1
    d, s, g = O.qt_quantize(O.QF_NF4, x, 0)
    assert s[0] == 1.0
    assert np.array_equal(O.qt_dequantize(O.QF_NF4, d, s, g, x.size), x)
    x = np.array([6.0, 0.25, 0.75, 5.0, -0.25, -6.0], np.float32)
    d, s, g = O.qt_quantize(O.QF_NVFP4, x, 0)
    assert s[0] == 1.0
    assert list(O.qt_dequantize(O.QF_NVFP4, d, s, g, 6)) == [6.0, 0.0, 0.5, 4.0, -0.0, -6.0]


def test_int4_odd_group_layout_kat():
    """n=6, group 3: each group packs on its own ([q0|q1<<4, q2] twice), while
    dequantize reads data[i/2] over the whole tensor (src/quantize.rs:380), so
    elements 3..5 read group 0's pad nibble and group 1's first two codes."""
    x = np.array([7.0, -7.0, 1.0, 3.5, 7.0, -3.5], np.float32)   # scales 1.0 and 1.0
    d, s, g = O.qt_quantize(O.QF_INT4, x, 3)
    assert g == 3 and list(s) == [1.0, 1.0]
    # codes: [7, -7, 1] -> 0x97, 0x01 ; [4 (3.5 rounds away), 7, -4] -> 0x74, 0x0C
    assert list(d) == [0x97, 0x01, 0x74, 0x0C]
    dq = O.qt_dequantize(O.QF_INT4, d, s, g, 6)
    # i=3 -> data[1] high nibble (pad 0); i=4 -> data[2] low (4); i=5 -> data[2] high (7)
    assert list(dq) == [7.0, -7.0, 1.0, 0.0, 4.0, 7.0]


def test_gguf_q4_negative_scale_kat():
    """Q4_0 divides by max/-8 (src/quantize.rs:174): the element of largest
    magnitude lands on -8 if positive, and on +8 -> 7 (saturated) if negative."""
    x = np.array([1.0, -2.0, 4.0, -8.0], np.float32)
    d, s, g = O.qt_quantize(O.QF_GGUF_Q4, x, 32)
    assert g == 32 and list(s) == [-1.0]          # block = min(32, 32), not n
    assert list(d) == [0x2F, 0x7C]
    assert list(O.qt_dequantize(O.QF_GGUF_Q4, d, s, g, 4)) == [1.0, -2.0, 4.0, -7.0]
    d, s, g = O.qt_quantize(O.QF_GGUF_Q4, -x, 32)
    assert list(O.qt_dequantize(O.QF_GGUF_Q4, d, s, g, 4)) == [-1.0, 2.0, -4.0, 8.0]


def test_dequant_scale_clamp_and_layouts():
    """scales[min(i/group, len-1)] (src/quantize.rs:326): a caller who shortens
    `scales` reuses the last one; GGUF blocks use min(group, 32)."""
    q = np.array([1, 2, 3, 4, 5, 6], np.int8).view(np.uint8)
    dq = O.qt_dequantize(O.QF_INT8, q, np.array([2.0], np.float32), 2, 6)
    assert list(dq) == [2.0, 4.0, 6.0, 8.0, 10.0, 12.0]
    assert O.qt_layout(O.QF_GGUF_Q8, 100, 0) == (100, 4, 32)
    assert O.qt_layout(O.QF_GGUF_Q4, 100, 64) == (50, 4, 32)
    assert O.qt_layout(O.QF_INT4, 7, 3) == (2 + 2 + 1, 3, 3)
    assert O.qt_layout(O.QF_FP16, 10, 32) == (20, 0, 0)


def test_linear_forward_within_gemm_bound():
    """QuantizedLinear::forward (src/quantize.rs:744-754) = dequantized W, then
    x.W^T + bias, within the f32 GEMM rounding bound of a float64 product."""
    rng = np.random.default_rng(8)
    m, k, n = 5, 96, 40
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    for f in ALL:
        d, s, g = O.qt_quantize(f, w, 32)
        wd = O.qt_dequantize(f, d, s, g, n * k).reshape(n, k).astype(np.float64)
        y = O.qt_linear_forward(f, x, d, s, g, n, b)
        exact = x.astype(np.float64) @ wd.T + b
        scale = np.abs(x.astype(np.float64)) @ np.abs(wd).T + np.abs(b)
        u = 2.0 ** -24
        assert np.all(np.abs(y - exact) <= (k + 2) * u * scale * 1.0001 + 1e-30)
