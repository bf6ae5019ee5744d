"""Pinning of the latent-attention (MLA) and rotary-encoding oracles.

* absorbed == materialised (reference tests/test_attention_xla.py:458-498):
  ``q W_K`` attended over the latent equals ``q`` attended over ``C W_K^T``;
* folded rows == unfolded (reference tests/test_latent_attention.py:828-858);
* absorbed == ``xla_attention`` over the latent broadcast to every head;
* the config-5 construction (absorbed NoPE part + shared RoPE part) equals
  plain per-head attention with materialised K = [C W_UK^T | rope(k_pe)],
  V = C W_UV^T;
* RoPE: norm-preserving, relative (``<R(m) q, R(n) k>`` depends on m - n),
  identity at position 0, closed-form inverse frequencies.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.latent import fold_heads, unfold_heads
from tests._helpers import rng_normal


@pytest.mark.parametrize("q_len", [1, 4])
def test_absorbed_equals_materialised(q_len):
    B, T, R, H, dk, dv = 2, 32, 24, 2, 16, 8
    cache, q = rng_normal(0, (B, T, R), (B, q_len, H, dk))
    wk, wv = rng_normal(1, (H, dk, R), (H, dv, R), scale=1 / math.sqrt(R))
    mask = oracle.KVLenMask(np.array([20, 32], np.int32))
    key, value = oracle.materialize_kv(cache, wk, wv, H)
    want = oracle.xla_attention(q, key, value, mask=mask, sm_scale=1 / math.sqrt(dk))
    got = oracle.xla_mla(q, cache, wk, wv, mask=mask)
    np.testing.assert_allclose(got, want, atol=2e-6)
    # the absorbed route explicitly
    q_lat = np.einsum("bqhd,hdr->bqhr", q, wk)
    o_lat = oracle.xla_mla(q_lat, cache, sm_scale=1 / math.sqrt(dk), mask=mask)
    np.testing.assert_allclose(np.einsum("bqhr,hdr->bqhd", o_lat, wv), want, atol=2e-6)


def test_absorbed_equals_broadcast_latent():
    q, cache = rng_normal(2, (2, 3, 4, 16), (2, 50, 16))
    got = oracle.xla_mla(q, cache)
    kv = np.broadcast_to(cache[:, :, None, :], (2, 50, 4, 16))
    np.testing.assert_allclose(got, oracle.xla_attention(q, kv, kv, sm_scale=0.25), atol=1e-6)


def test_fold_heads_row_order_and_equivalence():
    q, cache = rng_normal(3, (2, 3, 4, 16), (2, 40, 16))
    f = fold_heads(q)
    assert f.shape == (2, 12, 1, 16)
    np.testing.assert_array_equal(f[1, 2 * 4 + 3, 0], q[1, 2, 3])  # row = t*H + h
    mask = oracle.KVLenMask(np.array([40, 9], np.int32))
    a = oracle.xla_mla(q, cache, mask=mask)
    b = unfold_heads(oracle.xla_mla(f, cache, mask=mask, sm_scale=0.25), 3, 4)
    np.testing.assert_allclose(a, b, atol=1e-6)


def test_config5_construction_equals_materialised_mha():
    """[q_nope W_UK | rope(q_pe)] over [C | rope(k_pe)] then W_UV == per-head attention."""
    B, S, H, R, dn, dr, dv = 2, 30, 3, 16, 8, 4, 8
    c_kv, k_pe, q_nope, q_pe = rng_normal(4, (B, S, R), (B, S, dr), (B, 1, H, dn), (B, 1, H, dr))
    w_uk, w_uv = rng_normal(5, (H, dn, R), (H, dv, R), scale=0.3)
    kpos, qpos = np.arange(S), np.array([S])
    k_rot = oracle.apply_rotary(k_pe, kpos)
    q_rot = oracle.apply_rotary(q_pe, qpos)
    scale = 1 / math.sqrt(dn + dr)
    q_cat = np.concatenate([np.einsum("bqhd,hdr->bqhr", q_nope, w_uk), q_rot], -1)
    cache = np.concatenate([c_kv, k_rot], -1)
    o = oracle.xla_mla(q_cat, cache, sm_scale=scale)[..., :R]
    got = np.einsum("bqhr,hdr->bqhd", o, w_uv)
    key = np.concatenate([np.einsum("bsr,hdr->bshd", c_kv, w_uk),
                          np.broadcast_to(k_rot[:, :, None], (B, S, H, dr))], -1)
    val = np.einsum("bsr,hdr->bshd", c_kv, w_uv)
    q_full = np.concatenate([q_nope, q_rot], -1)
    want = oracle.xla_attention(q_full, key, val, sm_scale=scale)
    np.testing.assert_allclose(got, want, atol=2e-5)


def test_rope_invariants():
    (x,) = rng_normal(6, (5, 2, 8))
    pos = np.arange(5)
    r = oracle.apply_rotary(x, pos)
    np.testing.assert_allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)
    np.testing.assert_allclose(r[0], x[0], atol=1e-7)  # position 0: identity
    q, k = rng_normal(7, (1, 8), (1, 8))

    def dot(m, n):
        return float(np.dot(oracle.apply_rotary(q, [m])[0], oracle.apply_rotary(k, [n])[0]))

    assert dot(7, 3) == pytest.approx(dot(14, 10), rel=1e-4, abs=1e-5)
    assert dot(7, 3) != pytest.approx(dot(7, 4), rel=1e-3)


def test_rope_pair_rotation_closed_form():
    x = np.array([[1.0, 0.0, 0.0, 1.0]], np.float32)
    f = oracle.inv_freq(4)
    np.testing.assert_allclose(f, [1.0, 10000.0 ** -0.5], rtol=1e-6)
    r = oracle.apply_rotary(x, [2])
    a0, a1 = 2 * f[0], 2 * f[1]
    # interleaved pairs (x0, x1) -> (x0 cos - x1 sin, x1 cos + x0 sin)
    np.testing.assert_allclose(r[0], [math.cos(a0), math.sin(a0), -math.sin(a1), math.cos(a1)],
                               atol=1e-6)
