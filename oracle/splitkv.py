"""numpy restatement of the split-KV ("flash-decoding") forward (oracle).

Follows ``probjax/nn/pallas_kernels/kernels/attention_splitkv.py``:

* ``default_num_splits`` -- ``:106-118`` (target 2 x 82 programs, >= 256 keys
  per split, at least 2 splits when that allows)
* ``pack_queries`` / ``unpack_rows`` -- ``:121-134`` (row ``g * Lq + t``)
* ``splitkv_forward``    -- ``:137-250``: per split, exp2-domain online softmax
  with ``NEG_INF = -1e15`` for keys past the end (``:69-103``); each split's
  output normalised by its own sum and a base-2 LSE (``NEG_INF`` for an empty
  split); exact merge ``w = exp2(lse - max)``, ``O = sum w O_s / sum w``
  (``:236-245``); the returned LSE is natural-log (``:248-250``).

``kv_lengths`` (optional, ``[B]``) extends the restatement with the per-batch
key-length mask of ``KVLenMask`` (keys ``>= L[b]`` masked like keys past the
end): the reference split-KV kernel only runs unmasked
(``kernels/attention.py:2672-2675``), so with lengths this models the HIP
decode path's chunked kernel, whose semantics come from ``xla_attention`` +
``KVLenMask``.

Parity pinned (``tests/test_oracle_splitkv.py``): merge == unsplit
``xla_attention`` for every split count (reference
``tests/test_attention_gqa_splitkv.py:170-201``); pack/unpack round trip;
``default_num_splits`` table; LSE vs ``scipy.special.logsumexp``.
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import LOW_PRECISION, round_to

LOG2E = 1.4426950408889634
NEG_INF = -1e15
TARGET_PROGRAMS = 2 * 82
MIN_SPLIT_LEN = 256


def default_num_splits(batch, num_kv_heads, row_blocks, kv_len, block_k):
    """attention_splitkv.py:106-118."""
    programs = batch * num_kv_heads * row_blocks
    want = max(2, math.ceil(TARGET_PROGRAMS / programs))
    most = max(1, kv_len // max(MIN_SPLIT_LEN, block_k))
    return int(min(want, most))


def pack_queries(q, num_kv_heads):
    """``[B, Lq, Hq, D] -> [B, Hkv, G * Lq, D]`` (attention_splitkv.py:121-126)."""
    b, lq, hq, d = q.shape
    g = hq // num_kv_heads
    q = q.reshape(b, lq, num_kv_heads, g, d)
    return np.transpose(q, (0, 2, 3, 1, 4)).reshape(b, num_kv_heads, g * lq, d)


def unpack_rows(o, lq, num_heads):
    """Inverse of ``pack_queries`` (attention_splitkv.py:129-134)."""
    b, hkv, _, dv = o.shape
    g = num_heads // hkv
    o = o.reshape(b, hkv, g, lq, dv)
    return np.transpose(o, (0, 3, 1, 2, 4)).reshape(b, lq, num_heads, dv)


def split_partials(q, k, v, *, sm_scale, split_len, kv_lengths=None, dtype="f32"):
    """Per-split normalised outputs and base-2 LSEs (attention_splitkv.py:43-103).

    Returns ``o_part [B, Hkv, S, R, Dv]`` and ``lse_part [B, Hkv, S, R]``.
    """
    b, lq, hq, d = q.shape
    _, lkv, hkv, _ = k.shape
    qp = pack_queries(q, hkv).astype(np.float32)  # [B, Hkv, R, D]
    rows = qp.shape[2]
    ns = -(-lkv // split_len)
    lengths = np.full((b,), lkv) if kv_lengths is None else np.minimum(kv_lengths, lkv)
    kt = np.transpose(k, (0, 2, 1, 3)).astype(np.float32)  # [B, Hkv, Lkv, D]
    vt = np.transpose(v, (0, 2, 1, 3)).astype(np.float32)
    o_part = np.zeros((b, hkv, ns, rows, v.shape[-1]), np.float32)
    lse_part = np.zeros((b, hkv, ns, rows), np.float32)
    for s in range(ns):
        k0, k1 = s * split_len, min((s + 1) * split_len, lkv)
        qk = np.matmul(qp, np.swapaxes(kt[:, :, k0:k1], -1, -2)) * np.float32(
            sm_scale * LOG2E
        )
        valid = np.arange(k0, k1)[None, :] < lengths[:, None]  # [B, keys]
        qk = np.where(valid[:, None, None, :], qk, np.float32(NEG_INF))
        m = np.maximum(np.float32(NEG_INF), qk.max(axis=-1))
        # The reference loads masked K/V as zeros, so a split whose keys are all
        # masked contributes o = 0 with an LSE of about -1e15 (zero weight in the
        # merge).  Masked keys get weight exactly 0 here, which gives the same
        # merged result and also holds for masked keys whose V is not zero.
        p = np.where(valid[:, None, None, :], np.exp2(qk - m[..., None]), np.float32(0.0))
        l_ = p.sum(axis=-1)
        pv = round_to(p, dtype) if dtype in LOW_PRECISION else p
        o = np.matmul(pv, vt[:, :, k0:k1])
        safe_l = np.where(l_ == 0.0, 1.0, l_)
        o_part[:, :, s] = o / safe_l[..., None]
        lse_part[:, :, s] = np.where(l_ == 0.0, NEG_INF, m + np.log2(safe_l))
    return o_part, lse_part


def merge_partials(o_part, lse_part):
    """Exact LSE combine over splits (attention_splitkv.py:236-250).

    Returns ``(out [B, Hkv, R, Dv], lse_natural [B, Hkv, R])``.
    """
    m = np.max(lse_part, axis=2, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    w = np.exp2(lse_part - m)
    denom = np.sum(w, axis=2)
    out = np.einsum("bhsr,bhsrd->bhrd", w, o_part) / np.where(denom == 0, 1.0, denom)[
        ..., None
    ]
    with np.errstate(divide="ignore"):
        lse = (m[:, :, 0] + np.log2(denom)) / LOG2E
    return out, lse


def splitkv_forward(
    q, k, v, *, sm_scale, num_splits=None, block_k=64, kv_lengths=None,
    dtype="f32", return_lse=False,
):
    """``q [B, Lq, Hq, D]``, ``k/v [B, Lkv, Hkv, *]`` -> ``[B, Lq, Hq, Dv]``."""
    q, k, v = (round_to(np.asarray(x, np.float32), dtype) for x in (q, k, v))
    b, lq, hq, _ = q.shape
    lkv, hkv = k.shape[1], k.shape[2]
    if hq % hkv:
        raise ValueError(f"Hq={hq} must be a multiple of Hkv={hkv}.")
    if num_splits is None:
        rows = (hq // hkv) * lq
        block_r = max(16, 1 << (min(rows, 64) - 1).bit_length())
        num_splits = default_num_splits(b, hkv, -(-rows // block_r), lkv, block_k)
    split_len = -(-(-(-lkv // num_splits)) // block_k) * block_k
    o_part, lse_part = split_partials(
        q, k, v, sm_scale=sm_scale, split_len=split_len, kv_lengths=kv_lengths,
        dtype=dtype,
    )
    out, lse = merge_partials(o_part, lse_part)
    out = unpack_rows(out, lq, hq).astype(np.float32)
    out = round_to(out, dtype)
    if not return_lse:
        return out
    return out, lse.reshape(b, hkv, hq // hkv, lq).reshape(b, hq, lq).astype(np.float32)
