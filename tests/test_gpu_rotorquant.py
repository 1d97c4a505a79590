"""GPU parity: Cl(3,0) rotation matrices and RotorQuant quantize/dequantize
against the oracle -- reconstructions, codes and scales bit-exact (the
contract is codes bit-exact and reconstructions within 1e-5)."""
import numpy as np
import pytest

import oracle as O
import workloads as W
from test_gpu_int8 import assert_f32_equal, host, to_dev

pytestmark = pytest.mark.gpu


def test_rotation_matrices_parity(dev, hip):
    r = W.rotors(200, seed=3)
    r[5] = (1.0, 0.0, 0.0, 0.0)
    r[6] = (2.0, 0.5, -1.0, 0.25)  # non-unit rotor
    got = host(hip.rotation_matrices(to_dev(r, dev)))
    exp = np.stack([O.rotor_rotation_matrix(v) for v in r])
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("rows,dim,bits", [(1, 12, 4), (2, 10, 3), (5, 6, 4), (333, 128, 4),
                                           (64, 129, 8), (7, 1, 2), (50, 2, 5), (3, 130, 4),
                                           (4100, 128, 4), (9, 2688, 4), (37, 64, 4),
                                           (19, 256, 4), (8, 256, 8), (1, 64, 2),
                                           (5, 3001, 4), (2, 6000, 8)])
def test_rotorquant_parity(dev, hip, rows, dim, bits):
    x = W.activations(rows, dim, seed=rows + dim)
    x[0, : min(dim, 3)] = 0.0              # an all-zero group (skipped, src/quant.rs:189-191)
    if rows > 1:
        x[1] *= np.float32(1e-13)          # whole row below the 1e-12 threshold
    rot = W.rotors((dim + 2) // 3, seed=dim)
    y, codes, scales = hip.rotorquant_quantize(to_dev(x, dev), to_dev(rot, dev), bits,
                                               want_codes=True)
    ye, ce, se = O.rotorquant_quantize(x, rot, bits)
    assert np.array_equal(host(codes), ce)
    assert np.array_equal(host(scales), se)
    assert_f32_equal(host(y), ye)
    # y-only (the fused round trip the benchmark times) is identical
    y2, _, _ = hip.rotorquant_quantize(to_dev(x, dev), to_dev(rot, dev), bits)
    assert np.array_equal(host(y2), ye)
    # reconstruction from codes
    yd = hip.rotorquant_dequantize(codes, scales, dim, to_dev(rot, dev))
    assert_f32_equal(host(yd), O.rotorquant_dequantize(ce, se, dim, rot))


@pytest.mark.parametrize("dim", [128, 64])
def test_rotorquant_unaligned_generic_path(dev, hip, dim):
    """A tensor view that is only 4-byte aligned takes the generic per-group
    streaming kernel instead of the 16-byte tiled one; same results."""
    import torch
    rows = 45
    x = W.activations(rows, dim, seed=dim + 5)
    rot = W.rotors((dim + 2) // 3, seed=dim + 6)
    buf = to_dev(np.concatenate([np.zeros(1, np.float32), x.ravel()]), dev)
    xv = buf[1:].view(rows, dim)
    y = torch.empty(rows * dim + 1, dtype=torch.float32, device=dev)[1:].view(rows, dim)
    hip.rotorquant_quantize(xv, to_dev(rot, dev), 4, y=y)
    ye, _, _ = O.rotorquant_quantize(x, rot, 4)
    assert_f32_equal(host(y), ye)


def half_integer_cases(n_rows, bits, seed):
    """Rows of 3-groups whose quotient rv/scale sits exactly on, or within two
    ulps of, a half-integer k + 0.5 (identity rotors make rv = x): the cases
    where round-half-away-from-zero of the IEEE quotient is decided by the
    last bit. Scales are both exact (1.0) and inexact (random)."""
    g = W.rng(seed)
    qmax = np.float32(2 ** (bits - 1) - 1)
    groups = []
    for i in range(n_rows * 43):
        s = np.float32(1.0) if i % 4 == 0 else np.float32(g.uniform(1e-3, 10.0))
        m = np.float32(qmax * s)                       # max |rv|: scale = m / qmax ~= s
        scale = np.float32(m / qmax)
        k = int(g.integers(-int(qmax), int(qmax)))
        h = np.float32((np.float32(k) + np.float32(0.5)) * scale)
        for _ in range(int(g.integers(-2, 3))):        # walk 0..2 ulps either way
            h = np.nextafter(h, np.float32(np.inf) if k >= 0 else np.float32(-np.inf))
        if abs(h) > m:
            h = np.float32(np.sign(h) * m)
        c = np.float32(g.uniform(-1, 1) * m)
        groups.append((m if i % 2 else -m, h, c))
    x = np.array(groups, np.float32).reshape(n_rows, 43 * 3)[:, :128]
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("bits", [4, 8, 3])
def test_rotorquant_half_integer_quotients(dev, hip, bits):
    """The kernel rounds rv/scale through a reciprocal multiply and falls back
    to the exact division near half-integers; codes, scales and
    reconstructions must still equal the oracle's (true division + roundf)."""
    x = half_integer_cases(512, bits, seed=bits)
    rot = np.tile(np.array([1.0, 0.0, 0.0, 0.0], np.float32), (43, 1))
    y, codes, scales = hip.rotorquant_quantize(to_dev(x, dev), to_dev(rot, dev), bits,
                                               want_codes=True)
    ye, ce, se = O.rotorquant_quantize(x, rot, bits)
    assert np.array_equal(host(scales), se)
    assert np.array_equal(host(codes), ce)
    assert_f32_equal(host(y), ye)


def test_rotorquant_reference_bounded_error(dev, hip):
    # src/quant.rs:291-310 (data i*0.37-1.5, dim 12, 4 bits, error < 0.15*range) with
    # rotors from the build's seeded generator (the reference's come from rand's StdRng)
    dim = 12
    data = (np.arange(dim, dtype=np.float32) * np.float32(0.37) - np.float32(1.5))[None, :]
    rot = W.rotors(4, seed=123)
    y, _, _ = hip.rotorquant_quantize(to_dev(data, dev), to_dev(rot, dev), 4)
    y = host(y)
    assert np.abs(y - data).max() < 0.15 * (data.max() - data.min())
    assert np.array_equal(y, O.rotorquant_quantize(data, rot, 4)[0])


def test_rotorquant_kv_full_size_sampled(dev, hip):
    """BASELINE RotorQuant config: K and V [8, 32, 4096, 128] f32 ~ N(0,1) with 3
    channels x10, 4 bits: 4096 sampled rows of each tensor against the oracle,
    plus the per-group error bound |x - y| <= sqrt(3)*scale/2 on every row."""
    import torch
    c = W.ROTORQUANT
    shape = (c["batch"], c["heads"], c["seq"], c["head_dim"])
    dim, bits = c["head_dim"], c["bits"]
    ng = (dim + 2) // 3
    gen = torch.Generator(device=dev)
    for which, seed in (("K", 11), ("V", 12)):
        gen.manual_seed(seed)
        x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)
        ch = torch.as_tensor(W.kv_outlier_channels(dim, seed), device=dev)
        x[..., ch] *= 10.0
        rot = W.rotors(ng, seed=seed)
        rot_d = to_dev(rot, dev)
        y, _, _ = hip.rotorquant_quantize(x, rot_d, bits)
        rows = x.numel() // dim
        x2, y2 = x.view(rows, dim), y.view(rows, dim)
        pick = np.sort(W.rng(seed).choice(rows, 4096, replace=False))
        pidx = torch.as_tensor(pick, device=dev)
        xs = host(x2[pidx])
        ye, _, se = O.rotorquant_quantize(xs, rot, bits)
        assert_f32_equal(host(y2[pidx]), ye)
        # error bound on all rows, using the scales of a codes pass
        _, codes, scales = hip.rotorquant_quantize(x, rot_d, bits, want_y=False, want_codes=True)
        assert np.array_equal(host(scales[pidx]), se)
        pad = torch.zeros((rows, 3 * ng - dim), device=dev)
        d = (torch.cat([x2, pad], 1) - torch.cat([y2, pad], 1)).view(rows, ng, 3).norm(dim=2)
        bound = float(np.sqrt(3) * 0.5 * (1 + 1e-4)) * scales + 1e-6
        assert bool((d <= bound).all()), which
        assert int(codes.abs().max()) == 7
        del x, y, codes, scales, d
        torch.cuda.empty_cache()
