"""numpy restatement of flex_attention's low-rank bias folding (oracle) -- TEST INFRASTRUCTURE ONLY.

Follows ``probjax/nn/layers/attention.py``:

* ``split_low_rank_bias`` -- ``_split_low_rank_bias`` ``:1322-1345``: the
  ``LowRankBias`` / ``BatchedLowRankBias`` / ``LearnedAlibiBias`` terms of a
  bias or ``SumBias`` tree, and the remainder;
* ``fold_low_rank``       -- ``flex_attention`` ``:1600-1635``: K/V repeated
  to the query heads (GQA), each term's factors cast to the input dtype and
  scaled by ``sqrt(scale / sm_scale)`` appended to Q and K, zero features
  appended to V;
* ``flex_low_rank``       -- attention over the folded inputs (the XLA
  reference on them), output sliced to the value width;
* ``flex_low_rank_backward`` -- the VJP of that computation: the attention
  backward on the folded inputs, then the chain rule back through the
  concatenation, the scaling, the broadcasts of ``factors()`` and the GQA
  repeat (what JAX's autodiff of the folding computes).

Parity pinned (``tests/test_oracle_lowrank.py``): the reference's own tests
restated (``tests/test_learnable_attention_bias.py``: folded == dense bias
for output and factor gradients, low-rank terms extracted from a SumBias,
LearnedAlibiBias == ``-slope * (q - k)``); gradients against torch float64
autograd of the dense-bias formulation (independent of the folding), for
per-head, shared, per-example and learned-ALiBi factors, with GQA and a
causal mask.
"""

from __future__ import annotations

import math

import numpy as np

from .attention_xla import xla_attention
from .backward import attention_backward
from .bf16 import round_to
from .masks import BatchedLowRankBias, LearnedAlibiBias, LowRankBias, SumBias

_LOW_RANK = (LowRankBias, BatchedLowRankBias, LearnedAlibiBias)


def split_low_rank_bias(bias):
    """``(terms, remainder)`` (layers/attention.py:1322-1345)."""
    if bias is None:
        return [], None
    if isinstance(bias, _LOW_RANK):
        return [bias], None
    if isinstance(bias, SumBias):
        lt, lhs = split_low_rank_bias(bias.lhs)
        rt, rhs = split_low_rank_bias(bias.rhs)
        rest = rhs if lhs is None else lhs if rhs is None else SumBias(lhs, rhs)
        return lt + rt, rest
    return [], bias


def _cast(x, dtype):
    return round_to(np.asarray(x, np.float32), dtype)


def fold_low_rank(q, k, v, terms, sm_scale, dtype="f32"):
    """``(q', k', v')`` of the folding (layers/attention.py:1600-1635)."""
    if sm_scale <= 0:
        raise ValueError("LowRankBias requires a positive sm_scale")
    q, k, v = (_cast(x, dtype) for x in (q, k, v))
    hq = q.shape[2]
    if k.shape[2] != hq:
        rep = hq // k.shape[2]
        k, v = np.repeat(k, rep, axis=2), np.repeat(v, rep, axis=2)
    qx, kx = [], []
    for t in terms:
        uf, vf = t.factors(q.shape[1], k.shape[1], hq)
        f = math.sqrt(t.scale / sm_scale)
        qx.append(_cast(np.broadcast_to(_cast(uf, dtype), q.shape[:-1] + (t.rank,)) * np.float32(f), dtype))
        kx.append(_cast(np.broadcast_to(_cast(vf, dtype), k.shape[:-1] + (t.rank,)) * np.float32(f), dtype))
    extra = sum(x.shape[-1] for x in qx)
    q2 = np.concatenate([q, *qx], axis=-1)
    k2 = np.concatenate([k, *kx], axis=-1)
    v2 = np.concatenate([v, np.zeros(v.shape[:-1] + (extra,), np.float32)], axis=-1)
    return q2, k2, v2


def flex_low_rank(q, k, v, *, mask=None, bias=None, sm_scale=1.0, dtype="f32", compute_dtype=np.float32,
                  return_lse=False):
    """``flex_attention`` with the low-rank terms of ``bias`` folded."""
    terms, rest = split_low_rank_bias(bias)
    q2, k2, v2 = fold_low_rank(q, k, v, terms, sm_scale, dtype)
    o, lse = xla_attention(q2, k2, v2, mask=mask, bias=rest, sm_scale=sm_scale, strategy="dense",
                           dtype=dtype, compute_dtype=compute_dtype, return_lse=True)
    o = o[..., : np.shape(v)[-1]]
    return (o, lse) if return_lse else o


def _factor_grads(t, gq, gk, q_len, kv_len, num_heads, cdt):
    """Cotangents of a term's stored factors from those of its folded
    ``[B, L, H, rank]`` features (already multiplied by the fold scale)."""
    if isinstance(t, LearnedAlibiBias):
        qp = np.arange(q_len, dtype=cdt) + t.query_offset
        kp = np.arange(kv_len, dtype=cdt) + t.key_offset
        ds = -np.einsum("bqh,q->h", gq[..., 0], qp) + np.einsum("bkh,k->h", gk[..., 1], kp)
        return (ds.sum(keepdims=True) if t.slopes.shape[0] == 1 else ds,)
    if isinstance(t, LowRankBias):
        gu = gq.sum(axis=0).transpose(1, 0, 2)  # [H, q_len, r]
        gv = gk.sum(axis=0).transpose(1, 0, 2)
        if t.query_factors.shape[0] == 1:
            gu, gv = gu.sum(axis=0, keepdims=True), gv.sum(axis=0, keepdims=True)
        du = np.zeros(t.query_factors.shape, cdt)
        dv = np.zeros(t.key_factors.shape, cdt)
        du[:, :q_len] = gu
        dv[:, :kv_len] = gv
        return du, dv
    # BatchedLowRankBias: factors [B, L|1, r] broadcast over heads (and queries)
    gu, gv = gq.sum(axis=2), gk.sum(axis=2)
    du = np.zeros(t.query_factors.shape, cdt)
    dv = np.zeros(t.key_factors.shape, cdt)
    if t.query_factors.shape[1] == 1:
        du[:, 0] = gu.sum(axis=1)
    else:
        du[:, :q_len] = gu
    dv[:, :kv_len] = gv
    return du, dv


def flex_low_rank_backward(q, k, v, do, *, mask=None, bias=None, sm_scale=1.0, dtype="f32",
                           compute_dtype=np.float32, return_features=False):
    """``(dq, dk, dv, [factor cotangents per term])`` of ``flex_low_rank``
    (and, with ``return_features``, each term's folded-feature cotangents
    ``(gq, gk)``, ``[B, L, H, rank]``, scaled by the fold scale)."""
    cdt = np.dtype(compute_dtype).type
    terms, rest = split_low_rank_bias(bias)
    B, Lq, Hq, D = np.shape(q)
    Lk, Hkv, Dv = np.shape(k)[1], np.shape(k)[2], np.shape(v)[-1]
    q2, k2, v2 = fold_low_rank(q, k, v, terms, sm_scale, dtype)
    o, lse = xla_attention(q2, k2, v2, mask=mask, bias=rest, sm_scale=sm_scale, strategy="dense",
                           dtype=dtype, compute_dtype=compute_dtype, return_lse=True)
    do = _cast(do, dtype)
    do2 = np.concatenate([do, np.zeros(do.shape[:-1] + (v2.shape[-1] - Dv,), np.float32)], axis=-1)
    dq2, dk2, dv2 = attention_backward(q2, k2, v2, o, do2, lse, mask=mask, bias=rest, sm_scale=sm_scale,
                                       dtype=dtype, compute_dtype=compute_dtype)
    dq2, dk2, dv2 = (np.asarray(x, cdt) for x in (dq2, dk2, dv2))
    G = Hq // Hkv
    # the repeat's VJP sums each group's per-head gradients in the input dtype
    dk = _cast(dk2[..., :D].reshape(B, Lk, Hkv, G, D).sum(axis=3), dtype).astype(cdt)
    dv = _cast(dv2[..., :Dv].reshape(B, Lk, Hkv, G, Dv).sum(axis=3), dtype).astype(cdt)
    grads, feats, off = [], [], D
    for t in terms:
        f = cdt(math.sqrt(t.scale / sm_scale))
        gq = _cast(dq2[..., off : off + t.rank] * f, dtype).astype(cdt)
        gk = _cast(dk2[..., off : off + t.rank] * f, dtype).astype(cdt)
        grads.append(_factor_grads(t, gq, gk, Lq, Lk, Hq, cdt))
        feats.append((gq, gk))
        off += t.rank
    if return_features:
        return dq2[..., :D], dk, dv, grads, feats
    return dq2[..., :D], dk, dv, grads
