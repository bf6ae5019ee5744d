"""Pinning of the low-rank bias folding oracle (flex_attention,
layers/attention.py:1600-1635).

* The reference's own tests restated (tests/test_learnable_attention_bias.py):
  LowRankBias equals its explicit factor product; folding equals the dense
  bias for outputs and factor gradients; low-rank terms are extracted from a
  SumBias; LearnedAlibiBias equals ``-slope * (q - k)``.
* Gradients against torch float64 autograd of the dense-bias formulation
  (softmax(sm_scale q.k + scale U.V) V), which does not fold anything.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.lowrank import flex_low_rank, flex_low_rank_backward, split_low_rank_bias
from tests._helpers import rng_normal


def _inputs(seed=0, B=1, L=16, Hq=2, Hkv=2, D=8):
    return rng_normal(seed, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))


def test_low_rank_bias_matches_explicit_factor_product():
    """tests/test_learnable_attention_bias.py:48-53."""
    qf, kf = rng_normal(1, (2, 16, 3), (2, 16, 3))
    b = oracle.LowRankBias(qf, kf, scale=0.25)
    for h in range(2):
        got = b(np.zeros((16, 16), np.float32), h, np.arange(16), np.arange(16))
        np.testing.assert_allclose(got, 0.25 * qf[h] @ kf[h].T, atol=1e-6)


def test_learned_alibi_matches_causal_linear_distance():
    """tests/test_learnable_attention_bias.py:118-124."""
    slopes = np.array([0.5, 0.25], np.float32)
    b = oracle.LearnedAlibiBias(slopes)
    pos = np.arange(8)
    for h in range(2):
        got = b(np.zeros((8, 8), np.float32), h, pos, pos)
        np.testing.assert_allclose(got, -slopes[h] * (pos[:, None] - pos[None, :]), atol=1e-6)
    # the rank-2 factorisation reproduces it
    uf, vf = b.factors(8, 8, 2)
    np.testing.assert_allclose(np.einsum("qhr,khr->hqk", uf[0], vf[0])[1],
                               -slopes[1] * (pos[:, None] - pos[None, :]), atol=1e-5)


@pytest.mark.parametrize("which", ["low_rank", "shared_heads", "batched", "alibi", "sum"])
def test_folding_equals_dense_bias(which):
    """Folded into Q/K == the bias added to the scores (tests/
    test_learnable_attention_bias.py:56-86), here in float64 compute."""
    q, k, v, _ = _inputs(2, B=2)
    qf, kf = rng_normal(3, (2, 16, 3), (2, 16, 3))
    terms = {
        "low_rank": oracle.LowRankBias(qf, kf, scale=0.5),
        "shared_heads": oracle.LowRankBias(qf[:1], kf[:1], scale=0.5),
        "batched": oracle.BatchedLowRankBias.from_key_bias(rng_normal(4, (2, 16))[0]),
        "alibi": oracle.LearnedAlibiBias(np.array([0.5, 0.25], np.float32)),
        "sum": oracle.LowRankBias(qf, kf, scale=0.25) + oracle.CausalAlibiBias(),
    }
    bias = terms[which]
    mask = oracle.CausalMask() if which in ("alibi", "sum") else None
    got = flex_low_rank(q, k, v, mask=mask, bias=bias, sm_scale=1 / math.sqrt(8), compute_dtype=np.float64)
    want = oracle.xla_attention(q, k, v, mask=mask, bias=bias, sm_scale=1 / math.sqrt(8), strategy="dense",
                                compute_dtype=np.float64)
    np.testing.assert_allclose(got, want, atol=2e-6)
    lr, rest = split_low_rank_bias(bias)
    assert len(lr) == 1 and (rest is None) == (which != "sum")


def _torch_dense_grads(q, k, v, do, scale, bias_fn, params, causal):
    import torch

    tq, tk, tv = (torch.tensor(np.array(x), dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    tp = [torch.tensor(np.array(p), dtype=torch.float64, requires_grad=True) for p in params]
    G = q.shape[2] // k.shape[2]
    kk, vv = tk.repeat_interleave(G, dim=2), tv.repeat_interleave(G, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, kk) * scale + bias_fn(*tp)
    if causal:
        L = q.shape[1]
        s = s.masked_fill(~torch.tril(torch.ones(L, L, dtype=torch.bool)), float("-inf"))
    o = torch.einsum("bhqk,bkhd->bqhd", torch.softmax(s, -1), vv)
    (o * torch.tensor(do, dtype=torch.float64)).sum().backward()
    return o.detach().numpy(), [t.grad.numpy() for t in (tq, tk, tv, *tp)]


@pytest.mark.parametrize("which", ["low_rank", "shared_heads", "batched", "alibi"])
def test_folded_gradients_match_torch_dense_autograd(which):
    import torch

    B, L, Hq, Hkv, D = 2, 16, 4, 2, 8
    q, k, v, do = _inputs(5, B=B, Hq=Hq, Hkv=Hkv, D=D)
    scale = 1 / math.sqrt(D)
    qf, kf = rng_normal(6, (Hq, 20, 3), (Hq, 20, 3))  # factors longer than the sequence
    if which == "low_rank":
        bias = oracle.LowRankBias(qf, kf, scale=0.5)
        params = [qf, kf]
        fn = lambda u, w: 0.5 * torch.einsum("hqr,hkr->hqk", u[:, :L], w[:, :L])[None]  # noqa: E731
    elif which == "shared_heads":
        bias = oracle.LowRankBias(qf[:1], kf[:1], scale=2.0)
        params = [qf[:1], kf[:1]]
        fn = lambda u, w: 2.0 * torch.einsum("hqr,hkr->hqk", u[:, :L], w[:, :L])[None]  # noqa: E731
    elif which == "batched":
        key_bias = rng_normal(7, (B, L))[0]
        bias = oracle.BatchedLowRankBias.from_key_bias(key_bias)
        params = [bias.query_factors, bias.key_factors]
        fn = lambda u, w: torch.einsum("bqr,bkr->bqk", u.expand(B, L, 1), w)[:, None]  # noqa: E731
    else:
        slopes = np.array([0.5, 0.25, 0.125, 0.0625], np.float32)
        bias = oracle.LearnedAlibiBias(slopes, query_offset=3)
        params = [slopes]
        pos = torch.arange(L, dtype=torch.float64)
        fn = lambda s: -s[:, None, None] * ((pos + 3)[:, None] - pos[None, :])[None]  # noqa: E731
    causal = which == "alibi"
    mask = oracle.CausalMask() if causal else None
    want_o, want = _torch_dense_grads(q, k, v, do, scale, fn, params, causal)
    got_o = flex_low_rank(q, k, v, mask=mask, bias=bias, sm_scale=scale, compute_dtype=np.float64)
    np.testing.assert_allclose(got_o, want_o, atol=2e-6)
    dq, dk, dv, fg = flex_low_rank_backward(q, k, v, do, mask=mask, bias=bias, sm_scale=scale,
                                            compute_dtype=np.float64)
    got = [dq, dk, dv, *fg[0]]
    for i, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, (i, g.shape, w.shape)
        np.testing.assert_allclose(g, w, atol=5e-6 * max(1.0, float(np.abs(w).max())), err_msg=str(i))
