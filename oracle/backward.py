"""numpy restatement of probjax's attention backward (oracle) -- TEST INFRASTRUCTURE ONLY.

Follows ``probjax/nn/pallas_kernels/kernels/attention.py``:

* ``preprocess_delta``   -- ``_preprocess_backward_kernel`` ``:853-867``:
  ``delta = sum_d o * do`` in fp32, ``o`` as the forward stored it.
* ``attention_backward`` -- ``mha_backward_kernel`` ``:909-1160`` (scan #1 dK/dV
  ``:989-1052``, scan #2 dQ ``:1089-1150``) and its driver
  ``_mha_backward_raw`` ``:3505-3560``:

  - ``s = sm_scale * q.k`` (fp32) ``[+ bias]``, masked -> ``-inf`` (the kernel
    writes ``DEFAULT_MASK_VALUE``; ``exp2`` of it is 0 on every row that has a
    valid key);
  - ``p = exp(s - lse)``: the kernel's ``exp2(s * log2e - lse_2)`` with the
    base-2 residual ``lse_2 = lse * log2e``;
  - ``dp = do . v^T``; ``ds = p * (dp - delta) * sm_scale``;
  - ``dv = p^T . do`` with ``p`` cast to ``do``'s dtype (``:1042``),
    ``dk = ds^T . q`` and ``dq = ds . k`` with ``ds`` cast to q's / k's dtype
    (``:1051``, ``:1148``); fp32 accumulation;
  - GQA: per-query-head ``dk``/``dv`` in the input dtype, summed over each KV
    head's group in fp32 and cast (``_sum_gqa_group`` ``:2123-2128``);
  - the dense bias gets no cotangent (the custom VJP returns zeros for the
    bias leaves, ``:3262-3263``); ``return_dbias`` gives the gradient the
    reference's dense ``dot_product_attention`` path gives a bias tensor
    (``layers/attention.py:1293-1319``, autodiff of ``scores + bias``):
    ``p * (dp - delta)`` per score, the dS before the scale;
  - score modifiers (soft capping, per-head scale) multiply ``ds`` by their
    derivative at the pre-bias score (``:1051-1056``; ``grad_tile``).

Rows without a valid key: the forward's natural-log LSE is ``+inf`` there
(the XLA path's convention, ``attention_xla.py:420``), so ``p = 0`` and such
rows contribute nothing -- the gradient of the constant 0 output those rows
have in the XLA path.

bf16 / fp16 inputs are float32 arrays holding bfloat16 / float16 values with
``dtype="bf16"`` / ``"f16"`` (P and dS rounded to that dtype before their
products, as the reference's casts do).

Parity pinned (``tests/test_oracle_backward.py``) by: torch autograd in
float64 through an explicit masked softmax and through
``scaled_dot_product_attention`` (independent of this restatement); central
finite differences in float64 on tiny inputs; the closed forms
``sum_k dv = sum_q do`` over rows with a valid key, ``dq = 0`` for identical
keys, exact zeros for masked keys and empty rows; bf16 mode within the
reference's gradient tolerance of fp32 (``tests/test_attention.py:597-626``);
a planted variant without ``delta`` is rejected by the finite differences.
"""

from __future__ import annotations

import numpy as np

from .bf16 import LOW_PRECISION, round_to


def preprocess_delta(o, do, compute_dtype=np.float32):
    """``delta[b, h, q] = sum_d o * do`` (attention.py:853-867) -> ``[B, Hq, Lq]``."""
    cdt = np.dtype(compute_dtype).type
    d = np.sum(np.asarray(o, cdt) * np.asarray(do, cdt), axis=-1)  # [B, Lq, Hq]
    return np.ascontiguousarray(np.transpose(d, (0, 2, 1)))


def attention_backward(
    q,
    k,
    v,
    o,
    do,
    lse,
    *,
    mask=None,
    bias=None,
    sm_scale: float = 1.0,
    dtype: str = "f32",
    compute_dtype=np.float32,
    return_dbias: bool = False,
):
    """Gradients ``(dq, dk, dv)`` of the attention forward (and ``dbias``
    ``[B, Hq, Lq, Lk]`` per query head with ``return_dbias``).

    ``q/o/do [B, Lq, Hq, D]``, ``k/v [B, Lk, Hkv, D]``, ``lse [B, Hq, Lq]``
    natural log (``+inf`` for rows without a valid key).  ``mask`` is an
    oracle mask object (``tile_keep``), ``bias`` a ``DenseBias`` (``tile_add``).
    """
    low = dtype in LOW_PRECISION
    cdt = np.dtype(compute_dtype).type
    q, k, v, o, do = (round_to(np.asarray(x, np.float32), dtype) for x in (q, k, v, o, do))
    B, Lq, Hq, D = q.shape
    Lk, Hkv = k.shape[1], k.shape[2]
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} must be a multiple of kv heads {Hkv}")
    G = Hq // Hkv
    lse = np.asarray(lse, cdt)
    delta = preprocess_delta(o, do, cdt)
    span_q = np.arange(Lq, dtype=np.int32)
    span_k = np.arange(Lk, dtype=np.int32)

    dq = np.zeros((B, Lq, Hq, D), cdt)
    dbias = np.zeros((B, Hq, Lq, Lk), cdt) if return_dbias else None
    dk_h = np.zeros((B, Lk, Hq, D), cdt)
    dv_h = np.zeros((B, Lk, Hq, v.shape[-1]), cdt)
    for b in range(B):
        keep = None if mask is None else np.asarray(mask.tile_keep(b, span_q, span_k), bool)
        for h in range(Hq):
            kv = h // G
            qb, kb, vb, dob = (x.astype(cdt) for x in (q[b, :, h], k[b, :, kv], v[b, :, kv], do[b, :, h]))
            s = qb @ kb.T
            if sm_scale != 1.0:
                s = s * cdt(sm_scale)
            gf = None
            if bias is not None:
                gf = bias.grad_tile(s, b, h, 0, Lq, 0, Lk)
                s = bias.tile_add(s, b, h, 0, Lq, 0, Lk).astype(cdt, copy=False)
            if keep is not None:
                s = np.where(keep, s, -np.inf).astype(cdt, copy=False)
            p = np.exp(s - lse[b, h][:, None])
            dp = dob @ vb.T
            ds = p * (dp - delta[b, h][:, None])
            if dbias is not None:
                dbias[b, h] = ds  # d(scores + bias)/d(bias) = 1
            if sm_scale != 1.0:
                ds = ds * cdt(sm_scale)
            if gf is not None:
                ds = ds * np.asarray(gf, cdt)  # score-modifier derivative (:1051-1056)
            pc = round_to(p, dtype).astype(cdt) if low else p
            dsc = round_to(ds, dtype).astype(cdt) if low else ds
            dv_h[b, :, h] = pc.T @ dob
            dk_h[b, :, h] = dsc.T @ qb
            dq[b, :, h] = dsc @ kb

    def finish(x):
        x = np.asarray(x, np.float32)
        return round_to(x, dtype)

    dk_h, dv_h = finish(dk_h), finish(dv_h)
    dk = np.sum(dk_h.reshape(B, Lk, Hkv, G, D).astype(cdt), axis=3)
    dv = np.sum(dv_h.reshape(B, Lk, Hkv, G, dv_h.shape[-1]).astype(cdt), axis=3)
    if dbias is not None:
        return finish(dq), finish(dk), finish(dv), dbias
    return finish(dq), finish(dk), finish(dv)
