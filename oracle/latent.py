"""numpy restatement of the latent (MLA) attention CPU path (oracle).

Follows ``probjax/nn/pallas_kernels/kernels/latent_attention.py``:

* ``materialize_kv`` -- ``:396-410`` (``K = C W_K^T``, ``V = C W_V^T`` per head;
  ``None`` -> the latent itself)
* ``xla_mla``        -- ``_xla_mla`` ``:591-625``: the shared latent is one KV
  head; absorbed (``wk=None``) attends ``q`` over ``C`` with ``K = V = C``;
  with projections, absorb vs materialise is chosen by FLOP count
  (``:618-625``)
* ``mla``            -- argument checks and the default scale
  ``1 / sqrt(qk_head_dim)`` (``:679-701``)
* ``fold_heads`` / ``unfold_heads`` -- ``layers/latent_attention.py:458-469``
  (row ``i * H + h``)
* ``materialized_mla`` -- ``_materialized_mla`` ``:413-468``: ``mha`` over the
  materialised K/V with the head dims zero-padded to their common width,
  sliced to ``v_dim`` (the contract of the materialised kernel, reference
  ``tests/test_latent_attention.py:341-379``); K/V in the input dtype (the
  einsum's output dtype)
* ``materialized_mla_backward`` -- the custom VJP's backward ``:571-589``:
  the VJP of ``_materialized_mla`` (``mha``'s backward, then the einsums'
  ``dC = dK W_K + dV W_V``, ``dW_K = dK^T C``, ``dW_V = dV^T C``)

Parity pinned (``tests/test_oracle_latent.py``): absorbed == materialised
(``q W_K`` over ``C`` vs ``q`` over ``C W_K^T``; reference
``tests/test_attention_xla.py:458-498``), folded == unfolded rows (reference
``tests/test_latent_attention.py:828-858``), and absorbed == ``xla_attention``
over the latent broadcast to every head.  The materialised backward is pinned
against torch float64 autograd through the explicit projection and a masked
softmax, and by central finite differences on the reference's own test shape
(``tests/test_latent_attention.py:280-297``).
"""

from __future__ import annotations

import math

import numpy as np

from .attention_xla import xla_attention
from .bf16 import round_to


def materialize_kv(cache, wk, wv, num_heads):
    """latent_attention.py:396-410."""
    cache = np.asarray(cache, np.float32)
    if wk is None:
        key = np.broadcast_to(cache[..., None, :], cache.shape[:-1] + (num_heads, cache.shape[-1]))
    else:
        key = np.einsum("...sr,hdr->...shd", cache, wk)
    if wv is None:
        value = np.broadcast_to(cache[..., None, :], cache.shape[:-1] + (num_heads, cache.shape[-1]))
    else:
        value = np.einsum("...sr,hdr->...shd", cache, wv)
    return key, value


def xla_mla(q, cache, wk=None, wv=None, *, mask=None, bias=None, sm_scale=None, dtype="f32"):
    """CPU ``mla`` (latent_attention.py:591-625 with the checks of :679-701)."""
    q = np.asarray(q, np.float32)
    cache = np.asarray(cache, np.float32)
    if q.ndim != 4:
        raise ValueError(f"q must be rank 4 [B,Q,H,D], got shape {q.shape}")
    if cache.ndim != 3:
        raise ValueError(f"cache must be rank 3 [B,S,R], got shape {cache.shape}")
    if (wk is None) != (wv is None):
        raise ValueError("provide both wk and wv (materialized) or neither (absorbed)")
    if wk is None and q.shape[-1] != cache.shape[-1]:
        raise ValueError("absorbed mode (wk=None) requires qk_head_dim == kv_lora_rank")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    common = dict(mask=mask, bias=bias, sm_scale=sm_scale, dtype=dtype)
    shared = cache[:, :, None, :]
    if wk is None:
        return xla_attention(q, shared, shared, **common)
    q_len, kv_len, rank = q.shape[1], cache.shape[1], cache.shape[-1]
    dk, dv = wk.shape[1], wv.shape[1]
    materialized_cost = kv_len * rank * (dk + dv) + q_len * kv_len * (dk + dv)
    absorbed_cost = q_len * rank * (dk + dv) + 2 * q_len * kv_len * rank
    if absorbed_cost < materialized_cost:
        q_lat = np.einsum("bqhd,hdr->bqhr", q, wk)
        o_lat = xla_attention(q_lat, shared, shared, **common)
        return np.einsum("bqhr,hdr->bqhd", o_lat, wv)
    key, value = materialize_kv(cache, wk, wv, q.shape[-2])
    return xla_attention(q, key, value, **common)


def fold_heads(q):
    """``[B, Q, H, R] -> [B, Q*H, 1, R]`` (layers/latent_attention.py:458-469)."""
    b, nq, h, r = q.shape
    return q.reshape(b, nq * h, 1, r)


def unfold_heads(o, num_q, num_heads):
    """``[B, Q*H, 1, R] -> [B, Q, H, R]``."""
    b = o.shape[0]
    return o.reshape(b, num_q, num_heads, o.shape[-1])


def _round(x, dtype):
    return x if dtype == "f32" else round_to(np.asarray(x, np.float32), dtype)


def _pad_last(x, width):
    pad = width - x.shape[-1]
    return x if pad == 0 else np.concatenate([x, np.zeros(x.shape[:-1] + (pad,), x.dtype)], axis=-1)


def _materialized_operands(q, cache, wk, wv, dtype, compute_dtype):
    cdt = np.dtype(compute_dtype).type
    q, cache, wk, wv = (round_to(np.asarray(x, np.float32), dtype) for x in (q, cache, wk, wv))
    q, cache, wk, wv = (x.astype(cdt) for x in (q, cache, wk, wv))
    key = _round(np.einsum("bsr,hdr->bshd", cache, wk, optimize=True), dtype).astype(cdt)
    value = _round(np.einsum("bsr,hdr->bshd", cache, wv, optimize=True), dtype).astype(cdt)
    width = max(key.shape[-1], value.shape[-1])
    return q, cache, wk, wv, key, value, width


def materialized_mla(q, cache, wk, wv, *, mask=None, bias=None, sm_scale=None, dtype="f32",
                     compute_dtype=np.float32, return_lse=False):
    """``_materialized_mla`` (latent_attention.py:413-468) -> ``[B, Lq, H, v_dim]``
    (and the LSE ``[B, H, Lq]`` of the padded attention)."""
    q, cache, wk, wv, key, value, width = _materialized_operands(q, cache, wk, wv, dtype, compute_dtype)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    o, lse = xla_attention(_pad_last(q, width), _pad_last(key, width), _pad_last(value, width), mask=mask,
                           bias=bias, sm_scale=sm_scale, strategy="dense", dtype=dtype,
                           compute_dtype=compute_dtype, return_lse=True)
    o = o[..., : wv.shape[1]]
    return (o, lse) if return_lse else o


def materialized_mla_backward(q, cache, wk, wv, do, *, mask=None, bias=None, sm_scale=None, dtype="f32",
                              compute_dtype=np.float32):
    """Gradients ``(dq, dcache, dwk, dwv)`` of ``materialized_mla`` (the custom
    VJP's backward, latent_attention.py:571-589)."""
    from .backward import attention_backward

    cdt = np.dtype(compute_dtype).type
    q, cache, wk, wv, key, value, width = _materialized_operands(q, cache, wk, wv, dtype, compute_dtype)
    dk_dim, dv_dim = wk.shape[1], wv.shape[1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    qp, kp, vp = _pad_last(q, width), _pad_last(key, width), _pad_last(value, width)
    o, lse = xla_attention(qp, kp, vp, mask=mask, bias=bias, sm_scale=sm_scale, strategy="dense",
                           dtype=dtype, compute_dtype=compute_dtype, return_lse=True)
    do = _round(np.asarray(do, np.float32), dtype).astype(cdt)
    dqp, dkp, dvp = attention_backward(qp, kp, vp, o, _pad_last(do, width), lse, mask=mask, bias=bias,
                                       sm_scale=sm_scale, dtype=dtype, compute_dtype=compute_dtype)
    dK = np.asarray(dkp[..., :dk_dim], cdt)
    dV = np.asarray(dvp[..., :dv_dim], cdt)
    dcache = _round(np.einsum("bshd,hdr->bsr", dK, wk, optimize=True), dtype).astype(cdt) + \
        _round(np.einsum("bshd,hdr->bsr", dV, wv, optimize=True), dtype).astype(cdt)
    dwk = np.einsum("bshd,bsr->hdr", dK, cache, optimize=True)
    dwv = np.einsum("bshd,bsr->hdr", dV, cache, optimize=True)
    return (np.asarray(dqp[..., :dk_dim]), _round(dcache, dtype), _round(dwk, dtype), _round(dwv, dtype))
