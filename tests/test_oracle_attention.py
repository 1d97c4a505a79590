"""CPU pins of the oracle's Tensor::flash_attention restatement
(src/tensor.rs:618-672), which the RotorQuant KV-cache attention is checked
against:
- float64 softmax attention (scores, max-subtracted exponentials, weighted
  sum) within an error bound that a dropped rescale, a wrong max or a
  transposed operand exceeds by orders of magnitude;
- one-hot attention: a key whose score dominates returns its own value row
  (catches k/v or position mix-ups);
- equal scores: the output is the mean of the value rows;
- nq == skv is the reference's own signature; nq = 1 (a decode query) is the
  same loop with one row.
"""
import numpy as np
import pytest

import oracle as O


def attn64(q, k, v, scale):
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    return np.einsum("bij,bjd->bid", p / p.sum(axis=2, keepdims=True), v.astype(np.float64))


def bound(q, k, v, scale):
    u = 2.0 ** -24
    dim, skv = q.shape[2], k.shape[1]
    sabs = np.einsum("bid,bjd->bij", np.abs(q).astype(np.float64), np.abs(k).astype(np.float64))
    ds = (dim + 4) * u * scale * sabs.max(axis=2)             # score error per row
    vmax = np.abs(v).max(axis=(1, 2))[:, None, None]
    return (4 * ds[..., None] + (skv + 8) * u) * vmax * 2


@pytest.mark.parametrize("b,nq,skv,dim", [(2, 16, 16, 8), (1, 1, 300, 128), (3, 4, 77, 129),
                                           (1, 64, 64, 32)])
def test_flash_attention_vs_float64(b, nq, skv, dim):
    rng = np.random.default_rng(b * 100 + skv)
    q = rng.standard_normal((b, nq, dim)).astype(np.float32)
    k = rng.standard_normal((b, skv, dim)).astype(np.float32)
    v = rng.standard_normal((b, skv, dim)).astype(np.float32)
    scale = 1.0 / np.sqrt(dim)
    got = O.flash_attention(q, k, v, scale)
    err = np.abs(got - attn64(q, k, v, scale))
    assert np.all(err <= bound(q, k, v, scale))


def test_flash_attention_one_hot_and_uniform():
    rng = np.random.default_rng(7)
    dim, skv = 16, 40
    k = rng.standard_normal((1, skv, dim)).astype(np.float32) * 0.01
    v = rng.standard_normal((1, skv, dim)).astype(np.float32)
    q = np.zeros((1, 1, dim), np.float32)
    q[0, 0, 0] = 1000.0
    k[0, 23, 0] = 10.0                                      # score 10000 vs ~10
    assert np.array_equal(O.flash_attention(q, k, v, 1.0)[0, 0], v[0, 23])
    k1 = np.repeat(k[:, :1], skv, axis=1)                   # equal scores: mean of v
    got = O.flash_attention(q, k1, v, 1.0)[0, 0]
    assert np.allclose(got, v[0].astype(np.float64).mean(axis=0), rtol=0, atol=1e-5)


def test_flash_attention_empty_keys_is_zero():
    q = np.ones((1, 2, 4), np.float32)
    z = np.zeros((1, 0, 4), np.float32)
    assert np.array_equal(O.flash_attention(q, z, z, 1.0), np.zeros((1, 2, 4), np.float32))
