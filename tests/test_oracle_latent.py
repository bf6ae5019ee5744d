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


def _torch_materialized_grads(q, cache, wk, wv, do, keep, scale):
    """float64 torch autograd through C W^T, a masked softmax and P V."""
    import torch

    ts = [torch.tensor(np.array(x), dtype=torch.float64, requires_grad=True) for x in (q, cache, wk, wv)]
    tq, tc, twk, twv = ts
    key = torch.einsum("bsr,hdr->bshd", tc, twk)
    value = torch.einsum("bsr,hdr->bshd", tc, twv)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, key) * scale
    s = s.masked_fill(~torch.as_tensor(keep)[:, None], float("-inf"))
    o = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, dim=-1), value)
    (o * torch.tensor(do, dtype=torch.float64)).sum().backward()
    return o.detach().numpy(), [t.grad.numpy() for t in ts]


@pytest.mark.parametrize("mask_name", ["none", "causal", "kvlen"])
def test_materialized_backward_matches_torch_autograd(mask_name):
    """The reference's gradient test shape (tests/test_latent_attention.py:
    280-297: b=2, s=32, heads=4, head_dim=16, rank=8, v_dim=12)."""
    b, s, h, dk, r, dv = 2, 32, 4, 16, 8, 12
    q, cache, do = rng_normal(3, (b, s, h, dk), (b, s, r), (b, s, h, dv))
    wk, wv = rng_normal(4, (h, dk, r), (h, dv, r), scale=1 / math.sqrt(r))
    masks = {"none": (None, np.ones((b, s, s), bool)),
             "causal": (oracle.CausalMask(), np.broadcast_to(np.tril(np.ones((s, s), bool)), (b, s, s))),
             "kvlen": (oracle.KVLenMask(np.array([32, 9], np.int32)),
                       np.arange(s)[None, None, :] < np.array([32, 9])[:, None, None] + np.zeros((1, s, 1), int))}
    mask, keep = masks[mask_name]
    scale = 1 / math.sqrt(dk)
    want_o, want = _torch_materialized_grads(q, cache, wk, wv, do, keep, scale)
    # The oracle keeps K / V / O in the fp32 storage dtype of the reference's
    # f32 mode (its einsum and attention outputs are fp32 arrays), so it sits
    # within a few fp32 ulps of the float64 chain; a dropped term, a sign or a
    # transposed operand is off by orders of magnitude more.
    got_o = oracle.materialized_mla(q, cache, wk, wv, mask=mask, compute_dtype=np.float64)
    np.testing.assert_allclose(got_o, want_o, atol=1e-6)
    got = oracle.materialized_mla_backward(q, cache, wk, wv, do, mask=mask, compute_dtype=np.float64)
    for name, g, w in zip(("dq", "dcache", "dwk", "dwv"), got, want):
        assert g.shape == w.shape, name
        np.testing.assert_allclose(g, w, atol=2e-6 * max(1.0, float(np.max(np.abs(w)))), err_msg=name)


def test_materialized_backward_finite_differences():
    b, s, h, dk, r, dv = 1, 6, 2, 5, 3, 4
    q, cache, do = rng_normal(5, (b, s, h, dk), (b, s, r), (b, s, h, dv))
    wk, wv = rng_normal(6, (h, dk, r), (h, dv, r))
    mask = oracle.CausalMask()
    args = [np.asarray(x, np.float64) for x in (q, cache, wk, wv)]

    def loss(xs):
        o = oracle.materialized_mla(*xs, mask=mask, compute_dtype=np.float64)
        return float(np.sum(o * do))

    grads = oracle.materialized_mla_backward(*args, do, mask=mask, compute_dtype=np.float64)
    eps = 1e-3
    rng = np.random.default_rng(7)
    for i, g in enumerate(grads):
        for _ in range(4):
            idx = tuple(int(rng.integers(n)) for n in args[i].shape)
            up = [a.copy() for a in args]
            dn = [a.copy() for a in args]
            up[i][idx] += eps
            dn[i][idx] -= eps
            fd = (loss(up) - loss(dn)) / (2 * eps)
            # the forward stores fp32 (see above), so the step is large and the
            # bound covers its O(eps^2) truncation; planted mistakes are O(1e-1)
            assert abs(fd - g[idx]) <= 3e-3 * max(1.0, abs(fd)), (i, idx, fd, g[idx])


def test_materialized_bf16_close_to_f32():
    b, s, h, dk, r, dv = 2, 64, 2, 32, 48, 24
    q, cache, do = rng_normal(8, (b, s, h, dk), (b, s, r), (b, s, h, dv))
    wk, wv = rng_normal(9, (h, dk, r), (h, dv, r), scale=1 / math.sqrt(r))
    o32 = oracle.materialized_mla(q, cache, wk, wv, mask=oracle.CausalMask())
    o16 = oracle.materialized_mla(q, cache, wk, wv, mask=oracle.CausalMask(), dtype="bf16")
    assert np.max(np.abs(o32 - o16)) <= 3e-2
    g32 = oracle.materialized_mla_backward(q, cache, wk, wv, do, mask=oracle.CausalMask())
    g16 = oracle.materialized_mla_backward(q, cache, wk, wv, do, mask=oracle.CausalMask(), dtype="bf16")
    for a, c in zip(g32, g16):
        assert np.max(np.abs(a - c)) <= 3e-2 * max(1.0, np.max(np.abs(a)))
