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

Parity pinned (``tests/test_oracle_latent.py``): absorbed == materialised
(``q W_K`` over ``C`` vs ``q`` over ``C W_K^T``; reference
``tests/test_attention_xla.py:458-498``), folded == unfolded rows (reference
``tests/test_latent_attention.py:828-858``), and absorbed == ``xla_attention``
over the latent broadcast to every head.
"""

from __future__ import annotations

import math

import numpy as np

from .attention_xla import xla_attention


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
