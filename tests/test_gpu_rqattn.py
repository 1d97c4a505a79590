"""GPU parity of the RotorQuant KV cache (rnn_rotorquant_kv_pack) and the
attention that reads it (rnn_rotorquant_kv_attention): the result must equal
Tensor::flash_attention (src/tensor.rs:618-672) over the RotorQuant
reconstructions of K and V (the oracle's bit-exact dequantize, skipped
groups reconstructing to zero). The kernel scores from codes in the rotated
domain and sums in its own order, so the bar is a floating-point bound
around the float64 attention of the same K and V:
  |out - exact| <= (4 ds + (skv + 8) u) * max|V| * 2, ds = (dim + 16) u scale
  max_j sum_t |q_t| |K_jt| (the score error), u = 2^-24;
the oracle's own sequential restatement is held to the same bound."""
import numpy as np
import pytest

import oracle as O
import workloads as W

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def attn64(q, k, v, scale):
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    return np.einsum("bij,bjd->bid", p / p.sum(axis=2, keepdims=True), v.astype(np.float64))


def bound(q, k, v, scale):
    u = 2.0 ** -24
    dim, skv = q.shape[2], k.shape[1]
    sabs = np.einsum("bid,bjd->bij", np.abs(q).astype(np.float64), np.abs(k).astype(np.float64))
    ds = (dim + 16) * u * scale * sabs.max(axis=2)
    vmax = np.abs(v).max(axis=(1, 2))[:, None, None]
    return (4 * ds[..., None] + (skv + 8) * u) * vmax * 2


def make_cache(hip, dev, x, rot, bits, bh, seq, kind):
    """quantize x [bh*seq, dim] on the GPU, pack it as a K or V page; return
    (page, reconstruction)."""
    dim = x.shape[1]
    _, codes, scales = hip.rotorquant_quantize(to_dev(x, dev), to_dev(rot, dev), bits,
                                               want_y=False, want_codes=True)
    page = hip.rotorquant_kv_pack(codes, scales, bh, seq, dim, bits, kind)
    recon = O.rotorquant_dequantize(codes.cpu().numpy(), scales.cpu().numpy(), dim, rot)
    return page, recon.reshape(bh, seq, dim)


@pytest.mark.parametrize("bh,nq,seq,dim,bits", [(2, 1, 300, 128, 4), (3, 2, 64, 128, 4),
                                                (1, 1, 1, 128, 4), (4, 1, 129, 96, 3),
                                                (2, 3, 200, 130, 4), (1, 1, 4096, 128, 4),
                                                (2, 1, 70, 5, 2), (1, 4, 257, 192, 4),
                                                # past 64 groups: the wide kernel, one range
                                                (2, 1, 300, 193, 4), (3, 2, 130, 256, 3),
                                                (1, 1, 4096, 256, 4), (1, 3, 64, 576, 4),
                                                # several 256-group ranges, and past 64 KB of LDS
                                                (2, 1, 200, 800, 4), (1, 2, 70, 4096, 2),
                                                (1, 1, 100, 12000, 4),
                                                # few queries: the sequence split over workgroups
                                                (1, 1, 1000, 128, 4), (3, 1, 2000, 64, 3),
                                                (1, 2, 4096, 256, 4), (1, 1, 600, 800, 4),
                                                (1, 1, 513, 150, 2)])
def test_kv_attention_parity(dev, hip, bh, nq, seq, dim, bits):
    rng = np.random.default_rng(bh * 1000 + seq + dim)
    ng = (dim + 2) // 3
    kx = W.activations(bh * seq, dim, seed=seq + 1)
    kx[:, : max(1, dim // 40)] *= 10.0                      # outlier channels
    vx = W.activations(bh * seq, dim, seed=seq + 2)
    krot, vrot = W.rotors(ng, seed=dim + 3), W.rotors(ng, seed=dim + 4)
    kp, k = make_cache(hip, dev, kx, krot, bits, bh, seq, hip.RQ_PAGE_K)
    vp, v = make_cache(hip, dev, vx, vrot, bits, bh, seq, hip.RQ_PAGE_V)
    q = rng.standard_normal((bh, nq, dim)).astype(np.float32)
    scale = float(1.0 / np.sqrt(dim))
    out = hip.rotorquant_kv_attention(to_dev(q, dev), kp, vp, to_dev(krot, dev), to_dev(vrot, dev),
                                      seq, scale).cpu().numpy()
    exact = attn64(q, k, v, scale)
    lim = bound(q, k, v, scale)
    err = np.abs(out - exact)
    assert np.all(err <= lim), f"max err {err.max():.3g} (bound {lim.min():.3g})"
    ref = O.flash_attention(q, k, v, scale)                 # the reference's own order
    assert np.all(np.abs(ref - exact) <= lim)


def test_kv_attention_self_attention_signature(dev, hip):
    """nq == seq: the reference's flash_attention(q, k, v) shape [b, seq, d]."""
    bh, seq, dim = 2, 48, 64
    ng = (dim + 2) // 3
    x = W.activations(bh * seq, dim, seed=5)
    rot = W.rotors(ng, seed=6)
    kp, k = make_cache(hip, dev, x, rot, 4, bh, seq, hip.RQ_PAGE_K)
    vp, v = make_cache(hip, dev, x * 0.5, rot, 4, bh, seq, hip.RQ_PAGE_V)
    q = k.copy()
    out = hip.rotorquant_kv_attention(to_dev(q, dev), kp, vp, to_dev(rot, dev), to_dev(rot, dev),
                                      seq, 0.125).cpu().numpy()
    assert np.all(np.abs(out - attn64(q, k, v, 0.125)) <= bound(q, k, v, 0.125))


def test_kv_attention_empty_cache_and_errors(dev, hip):
    import torch
    q = torch.ones((2, 1, 128), device=dev)
    z16, z32 = torch.zeros(8, dtype=torch.int16, device=dev), torch.zeros(8, device=dev)
    rot = to_dev(W.rotors(43, seed=1), dev)
    out = hip.rotorquant_kv_attention(q, (z16, z32), (z16, z32), rot, rot, 0, 1.0)
    assert torch.equal(out, torch.zeros_like(out))          # row_sum 0 -> inv 0 (src/tensor.rs:657)
    big = 10 ** 6                                           # more LDS than a workgroup has
    rbig = torch.zeros(4 * ((big + 2) // 3), device=dev)
    with pytest.raises(hip.RnnError, match="LDS"):
        hip.rotorquant_kv_attention(torch.ones((1, 1, big), device=dev), (z16, z32), (z16, z32),
                                    rbig, rbig, 0, 1.0)
    codes = torch.zeros((4, 129), dtype=torch.int8, device=dev)
    with pytest.raises(hip.RnnError):                       # page kind must be K or V
        hip.rotorquant_kv_pack(codes, torch.zeros((4, 43), device=dev), 1, 4, 128, 4, 2)
    with pytest.raises(hip.RnnError):                       # 8-bit codes do not fit the page
        hip.rotorquant_kv_pack(codes, torch.zeros((4, 43), device=dev), 1, 4, 128, 8,
                               hip.RQ_PAGE_K)


def test_kv_attention_split_workspace_and_alloc(dev, hip):
    """The sequence split (two queries, 4096 positions): a caller's zeroed
    workspace (twice in a row: the calls leave its counts at zero), the
    wrapper's cached one and the library's own stream-ordered scratch (the
    plain entry point, called through ctypes) give the same bits; a
    workspace below the size the library asks for is refused."""
    import ctypes
    import torch
    bh, nq, seq, dim = 2, 1, 4096, 128
    ng = (dim + 2) // 3
    kp, _ = make_cache(hip, dev, W.activations(bh * seq, dim, seed=21), W.rotors(ng, seed=22), 4,
                       bh, seq, hip.RQ_PAGE_K)
    vp, _ = make_cache(hip, dev, W.activations(bh * seq, dim, seed=23), W.rotors(ng, seed=24), 4,
                       bh, seq, hip.RQ_PAGE_V)
    krot, vrot = to_dev(W.rotors(ng, seed=22), dev), to_dev(W.rotors(ng, seed=24), dev)
    q = torch.randn((bh, nq, dim), device=dev)
    need = hip.rotorquant_kv_attention_workspace_size(bh, nq, seq, dim)
    assert need > 0                                          # 2 queries do not fill the device
    ws = torch.zeros((need,), dtype=torch.uint8, device=dev)
    a = hip.rotorquant_kv_attention(q, kp, vp, krot, vrot, seq, 0.125, workspace=ws)
    a2 = hip.rotorquant_kv_attention(q, kp, vp, krot, vrot, seq, 0.125, workspace=ws)
    b = hip.rotorquant_kv_attention(q, kp, vp, krot, vrot, seq, 0.125)
    assert torch.equal(a, a2)
    q2 = torch.randn((bh, nq, dim), device=dev)               # another query, same workspace
    e = hip.rotorquant_kv_attention(q2, kp, vp, krot, vrot, seq, 0.125, workspace=ws)
    f = hip.rotorquant_kv_attention(q2, kp, vp, krot, vrot, seq, 0.125)
    assert torch.equal(e, f) and not torch.equal(a, e)
    c = torch.empty_like(a)
    P = ctypes.c_void_p
    rc = hip.load().rnn_rotorquant_kv_attention(
        P(q.data_ptr()), bh, nq, P(kp[0].data_ptr()), P(kp[1].data_ptr()), P(vp[0].data_ptr()),
        P(vp[1].data_ptr()), P(krot.data_ptr()), P(vrot.data_ptr()), seq, dim, 0.125,
        P(c.data_ptr()), P(torch.cuda.current_stream().cuda_stream))
    assert rc == hip.RNN_OK, hip.last_error()
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(a, c)
    with pytest.raises(hip.RnnError, match="workspace"):
        hip.rotorquant_kv_attention(q, kp, vp, krot, vrot, seq, 0.125, workspace=ws[: need - 4])
    assert hip.rotorquant_kv_attention_workspace_size(1024, 1, seq, dim) == 0  # queries fill it
