"""Mask / bias objects of the attention path, restated in numpy (oracle).

Restates ``probjax/nn/pallas_kernels/attention_mask_bias.py`` for the objects
the hot path uses:

* ``NoMask``         -- ``attention_mask_bias.py:583-612`` (all True, no block mask)
* ``CausalMask``     -- ``:615-646`` (``q >= k``, top-left aligned; block map
  ``kernel_utils/common.py:200-210``)
* ``QKVLengthMask``  -- ``:1077-1127`` (``(q < q_length) & (k < kv_length)``)
* ``KVLenMask``      -- ``:1399-1532`` (key ``k`` valid iff ``k < L[b]``; payload
  ``[B,1,1,1]`` one scalar per batch, ``:1487-1523``; no block mask)
* ``ComposeMask``    -- ``:324-525`` (and/or/xor; block-map combination rules
  ``:456-497``; at most one stateful child ``:359-371``)
* ``DenseBias``      -- ``:1807-1922`` (``scores + data``; ``[B|1, H|1, Q, K]``
  broadcast over size-1 batch/head, block index map ``:1849-1858``)
* ``SumBias``        -- ``:551-577`` (sum of additive deltas; derivative 1)
* positional masks   -- ``LocalWindowMask`` ``:651-704``, ``CausalLocalWindowMask``
  ``:707-750``, ``CausalFromBottomRightMask`` ``:753-782``, ``PrefixLMMask``
  ``:785-868``, ``SeqLenMask`` ``:1239-1398``
* segment masks      -- ``SameSegmentMask`` ``:1537-1668``, ``BlockDiagonalMask``
  ``:871-981``, ``BlockDiagonalCausalMask`` ``:984-1076``
* score modifiers    -- ``IdentityBias`` ``:2201-2220``, ``ConstantBias``
  ``:1781-1805``, ``CausalAlibiBias`` / ``SymmetricAlibiBias`` (slope
  ``2^-(h+1)``, ``:2223-2255, 2355-2380``), ``DistanceDecayBias``
  ``:2387-2414``, ``SoftCappingBias`` ``:2564-2603`` and ``PerHeadScaleBias``
  ``:2606-2648`` with their score derivatives (``grad_tile``)

The XLA reference evaluates a mask per ``(batch, head)`` on index tiles with
its payload sliced per batch (``attention_xla.py:227-279``); ``tile_keep``
below is that evaluation for one batch element, ``tile_add`` the bias one.

Parity pinned by the reference's own known-answer tests, restated in
``tests/test_oracle_masks.py`` (``tests/test_attention_mask_bias.py:54-209,
263-365`` in the reference) and by the equivalence
KVLenMask(L) == boolean key mask ``arange(S) < L`` == additive -inf bias.
``PerHeadScaleBias``'s derivative is the modifier's own (``scales[h]``), the
gradient of the XLA path; the Pallas kernels call ``grad`` with the batch
index in the head slot (``kernels/attention.py:1051-1056``).
"""

from __future__ import annotations

import numpy as np


def _cdiv(a: int, b: int) -> int:
    return -(-a // b)


class AttentionMask:
    """Base: ``__call__(q_idx, k_idx, seg_q, seg_k) -> bool[Q, K]``."""

    stateful = False
    query_independent = False

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):  # pragma: no cover
        raise NotImplementedError

    def tile_keep(self, b: int, span_q, span_k):
        """Mask of one ``[bq, kc]`` tile of batch ``b`` (attention_xla.py:247-268)."""
        return np.broadcast_to(
            self(span_q, span_k), (len(span_q), len(span_k))
        )

    def block_mask(self, q_len, kv_len, block_q, block_k):
        """``[nQ, nK]`` map of tiles that are not fully masked (generic fallback,
        attention_mask_bias.py:160-186: evaluate every tile)."""
        nq, nk = _cdiv(q_len, block_q), _cdiv(kv_len, block_k)
        bm = np.ones((nq, nk), dtype=bool)
        for i in range(0, q_len, block_q):
            for j in range(0, kv_len, block_k):
                rows = np.arange(i, i + block_q, dtype=np.int32)
                cols = np.arange(j, j + block_k, dtype=np.int32)
                if not np.asarray(self(rows, cols)).any():
                    bm[i // block_q, j // block_k] = False
        return bm

    def dense(self, q_len, kv_len, *, batch_size=1, num_heads=1):
        """``[B, H, Q, K]`` boolean mask (attention_mask_bias.py:65-101)."""
        q_idx = np.arange(q_len, dtype=np.int32)
        k_idx = np.arange(kv_len, dtype=np.int32)
        out = np.stack(
            [self.tile_keep(b, q_idx, k_idx) for b in range(batch_size)]
        )
        return np.broadcast_to(out[:, None], (batch_size, num_heads, q_len, kv_len))

    def __and__(self, other):
        return ComposeMask("and", self, other)

    def __or__(self, other):
        return ComposeMask("or", self, other)

    def __xor__(self, other):
        return ComposeMask("xor", self, other)

    def __invert__(self):
        return NotMask(self)


class NoMask(AttentionMask):
    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        return np.ones((len(q_idx), len(k_idx)), dtype=bool)

    def block_mask(self, q_len, kv_len, block_q, block_k):
        return None


class CausalMask(AttentionMask):
    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        return q_idx[:, None] >= k_idx[None, :]

    def block_mask(self, q_len, kv_len, block_q, block_k):
        # kernel_utils/common.py:200-210
        i = np.arange(_cdiv(q_len, block_q))
        j = np.arange(_cdiv(kv_len, block_k))
        i1 = np.minimum((i + 1) * block_q - 1, q_len - 1)
        j0 = j * block_k
        return j0[None, :] <= i1[:, None]


class QKVLengthMask(AttentionMask):
    def __init__(self, q_length: int, kv_length: int, block_sparse: bool = True):
        self.q_length, self.kv_length = int(q_length), int(kv_length)
        self.block_sparse = block_sparse

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        return (q_idx[:, None] < self.q_length) & (k_idx[None, :] < self.kv_length)

    def block_mask(self, q_len, kv_len, block_q, block_k):
        # attention_mask_bias.py:1103-1119
        if not self.block_sparse:
            return None
        bm = np.ones((_cdiv(q_len, block_q), _cdiv(kv_len, block_k)), dtype=bool)
        bm[(self.q_length - 1) // block_q + 1 :, :] = False
        bm[:, (self.kv_length - 1) // block_k + 1 :] = False
        return bm


class KVLenMask(AttentionMask):
    stateful = True
    query_independent = True

    def __init__(self, kv_lengths):
        self.kv_lengths = np.asarray(kv_lengths, dtype=np.int32).reshape(-1)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        if seg_q is not None or seg_k is not None:
            # attention_mask_bias.py:1455-1465: the per-batch payload is given.
            L = seg_k if seg_k is not None else seg_q
            valid_k = k_idx < np.asarray(L)
            return np.broadcast_to(valid_k[None, :], (len(q_idx), len(k_idx)))
        # :1467-1474 -- no payload: per-batch [B, Q, K]
        valid_k = k_idx[None, :] < self.kv_lengths[:, None]
        return np.broadcast_to(
            valid_k[:, None, :], (len(self.kv_lengths), len(q_idx), len(k_idx))
        )

    def get_data(self):
        # attention_mask_bias.py:1515-1523: payload [B, 1, 1, 1]
        return self.kv_lengths.reshape(-1, 1, 1, 1), None

    def tile_keep(self, b, span_q, span_k):
        # The XLA path slices the payload block of batch b, windows it down to a
        # scalar and feeds it as seg_q/seg_k (attention_xla.py:250-268, 146-168).
        L = self.kv_lengths[b]
        return self(span_q, span_k, L, L)

    def block_mask(self, q_len, kv_len, block_q, block_k):
        return None


class LocalWindowMask(AttentionMask):
    """attention_mask_bias.py:651-704: ``-right <= q - k <= left`` (right None -> 0)."""

    def __init__(self, left_window: int, right_window=None):
        self.left_window = int(left_window)
        self.right_window = right_window

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        d = np.asarray(q_idx)[:, None] - np.asarray(k_idx)[None, :]
        rw = 0 if self.right_window is None else int(self.right_window)
        return (d >= -rw) & (d <= self.left_window)


class CausalLocalWindowMask(AttentionMask):
    """:707-750: ``0 <= q - k <= left``."""

    def __init__(self, left_window: int):
        self.left_window = int(left_window)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        d = np.asarray(q_idx)[:, None] - np.asarray(k_idx)[None, :]
        return (d >= 0) & (d <= self.left_window)


class CausalFromBottomRightMask(AttentionMask):
    """:753-782: ``q + (kv_length - q_length) >= k``."""

    def __init__(self, q_length: int, kv_length: int):
        self.q_length, self.kv_length = int(q_length), int(kv_length)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        shift = self.kv_length - self.q_length
        return (np.asarray(q_idx)[:, None] + shift) >= np.asarray(k_idx)[None, :]


class PrefixLMMask(AttentionMask):
    """:785-868: ``(k < P) | (q >= k)``; ``prefix_lengths`` a scalar or ``[B]``
    (the kernel reads one value per batch element)."""

    stateful = True

    def block_mask(self, q_len, kv_len, block_q, block_k):
        return None  # per-batch data: no static tile map

    def __init__(self, prefix_lengths):
        self.prefix_lengths = np.asarray(prefix_lengths, dtype=np.int32)

    def _p(self, b):
        p = self.prefix_lengths
        return int(p) if p.ndim == 0 else int(p.reshape(-1)[b])

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        p = self._p(0) if seg_q is None else int(np.asarray(seg_q).reshape(-1)[0])
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        return (k_idx[None, :] < p) | (q_idx[:, None] >= k_idx[None, :])

    def tile_keep(self, b, span_q, span_k):
        return self(span_q, span_k, np.int32(self._p(b)))


class SeqLenMask(AttentionMask):
    """:1239-1398: inside the valid length ``L[b]`` full attention, outside it
    only the diagonal: ``(q < L & k < L) | (q == k)``."""

    stateful = True

    def block_mask(self, q_len, kv_len, block_q, block_k):
        return None  # per-batch data: no static tile map

    def __init__(self, seq_lengths):
        self.seq_lengths = np.asarray(seq_lengths, dtype=np.int32).reshape(-1)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        L = int(self.seq_lengths[0]) if seg_q is None else int(np.asarray(seg_q).reshape(-1)[0])
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        rect = (q_idx[:, None] < L) & (k_idx[None, :] < L)
        return rect | (q_idx[:, None] == k_idx[None, :])

    def tile_keep(self, b, span_q, span_k):
        return self(span_q, span_k, np.int32(self.seq_lengths[b]))


class SameSegmentMask(AttentionMask):
    """:1537-1668: ``seg_q[q] == seg_k[k]``; ids ``[B, L]`` or shared ``[L]``;
    keys use the query ids when ``key_segment_ids`` is None."""

    stateful = True

    def block_mask(self, q_len, kv_len, block_q, block_k):
        return None  # per-batch data: no static tile map

    def __init__(self, query_segment_ids, key_segment_ids=None):
        self.query_segment_ids = np.asarray(query_segment_ids, dtype=np.int32)
        self.key_segment_ids = None if key_segment_ids is None else np.asarray(key_segment_ids, np.int32)

    @staticmethod
    def _row(ids, b):
        return ids if ids.ndim == 1 else ids[b]

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        sq = self.query_segment_ids if seg_q is None else np.asarray(seg_q)
        kids = self.key_segment_ids if self.key_segment_ids is not None else self.query_segment_ids
        sk = kids if seg_k is None else np.asarray(seg_k)
        return sq[..., :, None] == sk[..., None, :]

    def tile_keep(self, b, span_q, span_k):
        kids = self.key_segment_ids if self.key_segment_ids is not None else self.query_segment_ids
        sq = self._row(self.query_segment_ids, b)[np.asarray(span_q)]
        sk = self._row(kids, b)[np.asarray(span_k)]
        return sq[:, None] == sk[None, :]


class BlockDiagonalMask(SameSegmentMask):
    """:871-981: same block id (the ids are segment ids)."""

    def __init__(self, query_block_ids, key_block_ids=None):
        super().__init__(query_block_ids, key_block_ids)


class BlockDiagonalCausalMask(SameSegmentMask):
    """:984-1076: same block id and ``q >= k``."""

    def __init__(self, query_block_ids, key_block_ids=None):
        super().__init__(query_block_ids, key_block_ids)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        same = super().__call__(q_idx, k_idx, seg_q, seg_k)
        return same & (np.asarray(q_idx)[:, None] >= np.asarray(k_idx)[None, :])

    def tile_keep(self, b, span_q, span_k):
        same = super().tile_keep(b, span_q, span_k)
        return same & (np.asarray(span_q)[:, None] >= np.asarray(span_k)[None, :])


class KeyPaddingMask(AttentionMask):
    """:1132-1236: keys ``k < count`` with a count per query row.

    ``__call__`` (:1143-1164): a scalar payload holds for every row; a vector
    ``kl`` gives row ``i`` the keys ``k < kl[i]``.  ``tile_keep`` follows the
    XLA path: ``get_data`` (:1192-1204) shapes a ``[T]`` payload as
    ``[1, T, 1, 1]`` (shared by every batch) and ``[B, T]`` as
    ``[B, T, 1, 1]``; the query block spec (:1175-1190) and
    ``_mask_data_window`` (attention_xla.py:146-168, 250-268) window it over
    query positions, zero-filled past ``T`` (attention_xla.py:130-133).  So
    row ``q`` of batch ``b`` keeps ``k < kl[q]`` (or ``kl[b, q]``) and rows
    ``q >= T`` keep nothing.  A boolean payload compares as 0/1.
    """

    stateful = True

    def __init__(self, key_lengths):
        self.key_lengths = np.asarray(key_lengths)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        kl = np.asarray(seg_q if seg_q is not None else self.key_lengths)
        k_idx = np.asarray(k_idx)
        if kl.ndim == 0:
            return np.broadcast_to(k_idx[None, :] < kl, (len(q_idx), len(k_idx)))
        if kl.ndim != 1:
            raise ValueError("KeyPaddingMask.__call__ takes a scalar or per-row vector payload")
        valid = k_idx[None, :] < kl.astype(np.int64)[:, None]
        return valid[: len(q_idx), :]

    def rows(self, b, span_q):
        """The count of each query row in ``span_q`` of batch ``b``."""
        kl = self.key_lengths.astype(np.int64)
        span_q = np.asarray(span_q)
        if kl.ndim == 0:
            return np.full(len(span_q), kl)
        vec = kl if kl.ndim == 1 else kl[b]
        padded = np.zeros(int(span_q.max()) + 1 if len(span_q) else 0, np.int64)
        n = min(len(vec), len(padded))
        padded[:n] = vec[:n]
        return padded[span_q]

    def tile_keep(self, b, span_q, span_k):
        return self(span_q, span_k, seg_q=self.rows(b, span_q))


class NotMask(AttentionMask):
    """:530-548: the complement of ``inner``."""

    def __init__(self, inner):
        self.inner = inner
        self.stateful = inner.stateful

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        return np.logical_not(self.inner(q_idx, k_idx, seg_q, seg_k))

    def tile_keep(self, b, span_q, span_k):
        return np.logical_not(self.inner.tile_keep(b, span_q, span_k))


def _payload_rows(vec2d_or_1d, b, span):
    """A ``[T]`` or ``[B, T]`` per-position payload read at positions ``span``
    of batch ``b``, zero past ``T`` (the XLA path's windowing of a
    ``[1|B, T, 1, 1]`` payload, attention_xla.py:130-133, 146-168)."""
    p = np.asarray(vec2d_or_1d)
    vec = p if p.ndim == 1 else p[b]
    span = np.asarray(span)
    out = np.zeros(len(span), vec.dtype)
    ok = span < len(vec)
    out[ok] = vec[span[ok]]
    return out


class MarginalizationMask(AttentionMask):
    """:1671-1778: ``(m[q] & m[k]) | (q == k)``.  ``tile_keep`` reads the
    payload (``get_data``: ``[T]`` shared by every batch, ``[B, T]`` per
    batch) at the query and at the key positions, as the XLA path does (the
    key ids default to the query payload, attention_xla.py:262-263)."""

    stateful = True

    def __init__(self, mask):
        self.mask = np.asarray(mask, bool)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        q_idx, k_idx = np.asarray(q_idx), np.asarray(k_idx)
        mq = np.asarray(seg_q, bool) if seg_q is not None else self.mask[..., q_idx]
        mk = np.asarray(seg_k, bool) if seg_k is not None else self.mask[..., k_idx]
        return (mq[..., :, None] & mk[..., None, :]) | (q_idx[:, None] == k_idx[None, :])

    def tile_keep(self, b, span_q, span_k):
        return self(span_q, span_k, _payload_rows(self.mask, b, span_q), _payload_rows(self.mask, b, span_k))


class ComposeMask(AttentionMask):
    def __init__(self, op: str, lhs: AttentionMask, rhs: AttentionMask):
        if op not in ("and", "or", "xor"):
            raise ValueError(f"Unknown op for ComposeMask: {op}")
        if lhs.stateful and rhs.stateful:
            raise ValueError("Cannot compose two stateful masks")
        self.op, self.lhs, self.rhs = op, lhs, rhs
        self.stateful = lhs.stateful or rhs.stateful
        self.query_independent = lhs.query_independent and rhs.query_independent

    def _combine(self, a, c):
        if self.op == "and":
            return np.logical_and(a, c)
        if self.op == "or":
            return np.logical_or(a, c)
        return np.logical_xor(a, c)

    def __call__(self, q_idx, k_idx, seg_q=None, seg_k=None):
        return self._combine(
            self.lhs(q_idx, k_idx, seg_q, seg_k), self.rhs(q_idx, k_idx, seg_q, seg_k)
        )

    def tile_keep(self, b, span_q, span_k):
        return self._combine(
            self.lhs.tile_keep(b, span_q, span_k), self.rhs.tile_keep(b, span_q, span_k)
        )

    def block_mask(self, q_len, kv_len, block_q, block_k):
        # attention_mask_bias.py:456-497 (stateful children are "unknown")
        def child(m):
            return None if m.stateful else m.block_mask(q_len, kv_len, block_q, block_k)

        lb, rb = child(self.lhs), child(self.rhs)
        if self.op == "and":
            if lb is not None and rb is not None:
                return np.asarray(lb) & np.asarray(rb)
            return lb if lb is not None else rb
        if lb is not None and rb is not None:
            return (np.asarray(lb) | np.asarray(rb)) if self.op == "or" else (
                np.asarray(lb) ^ np.asarray(rb)
            )
        return None


class AttentionBias:
    """Base: ``__call__(scores, h_idx, q_idx, k_idx, data) -> scores``."""

    def __add__(self, other):
        return SumBias(self, other)

    def tile_add(self, scores, b, h, q0, bq, k0, kc):
        """The bias evaluated on one score tile (attention_xla.py:227-246)."""
        return self(scores, h, np.arange(q0, q0 + bq), np.arange(k0, k0 + kc))

    def grad_tile(self, scores, b, h, q0, bq, k0, kc):
        """d(modified score)/d(score) on a tile: 1 for additive biases
        (attention_mask_bias.py:286-298)."""
        return np.ones_like(scores)


class DenseBias(AttentionBias):
    def __init__(self, bias):
        bias = np.asarray(bias, dtype=np.float32)
        if bias.ndim != 4:
            raise ValueError("bias must have shape [B|1, H|1, Q, K]")
        self.bias = bias

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        # attention_mask_bias.py:1822-1847
        if data is not None:
            return scores + data
        B, H = self.bias.shape[:2]
        if B != 1:
            raise ValueError(
                "DenseBias.__call__ without block data requires bias batch dimension to be 1"
            )
        hsel = 0 if H == 1 else int(h_idx)
        return scores + self.bias[0, hsel][np.asarray(q_idx)][:, np.asarray(k_idx)]

    def tile_add(self, scores, b, h, q0, bq, k0, kc):
        # Block index map (attention_mask_bias.py:1849-1858) evaluated at the XLA
        # path's grid point (0, b, h): batch/head 0 when the bias broadcasts.
        bb = b if self.bias.shape[0] != 1 else 0
        hh = h if self.bias.shape[1] != 1 else 0
        chunk = self.bias[bb, hh, q0 : q0 + bq, k0 : k0 + kc]
        if chunk.shape != (bq, kc):  # ragged tile: zero-padded (attention_xla.py:130-133)
            pad = np.zeros((bq, kc), np.float32)
            pad[: chunk.shape[0], : chunk.shape[1]] = chunk
            chunk = pad
        return self(scores, h, None, None, data=chunk)

    def dense(self, q_len, kv_len, *, batch_size=1, num_heads=1):
        # attention_mask_bias.py:1878-1905
        b = self.bias
        if b.shape[-2:] != (q_len, kv_len):
            raise ValueError(
                f"DenseBias shape mismatch: bias[...,Q,K]={b.shape[-2:]} vs ({q_len},{kv_len})"
            )
        if b.shape[0] not in (1, batch_size):
            raise ValueError(f"Cannot broadcast bias batch dim {b.shape[0]} to {batch_size}")
        if b.shape[1] not in (1, num_heads):
            raise ValueError(f"Cannot broadcast bias head dim {b.shape[1]} to {num_heads}")
        return np.broadcast_to(b, (batch_size, num_heads, q_len, kv_len))


class IdentityBias(AttentionBias):
    """attention_mask_bias.py:2201-2227."""

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        return scores


class ConstantBias(AttentionBias):
    """:1781-1805: ``scores + value``."""

    def __init__(self, value: float):
        self.value = float(value)

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        return scores + np.float32(self.value)


def alibi_slope(h: int) -> float:
    """:2223-2227: ``2^-(h+1)``."""
    return float(2.0 ** (-(int(h) + 1.0)))


class CausalAlibiBias(AttentionBias):
    """:2230-2255: ``scores - slope(h) * relu(q - k)``."""

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        d = np.maximum(np.asarray(q_idx)[:, None] - np.asarray(k_idx)[None, :], 0)
        return scores - np.float32(alibi_slope(h_idx)) * d.astype(np.float32)


class SymmetricAlibiBias(AttentionBias):
    """:2355-2380: ``scores - slope(h) * |q - k|``."""

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        d = np.abs(np.asarray(q_idx)[:, None] - np.asarray(k_idx)[None, :])
        return scores - np.float32(alibi_slope(h_idx)) * d.astype(np.float32)


class DistanceDecayBias(AttentionBias):
    """:2387-2414: ``scores - alpha * |q - k|``."""

    def __init__(self, alpha: float = 1.0):
        self.alpha = float(alpha)

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        d = np.abs(np.asarray(q_idx)[:, None] - np.asarray(k_idx)[None, :]).astype(np.float32)
        return scores - np.float32(self.alpha) * d


class SoftCappingBias(AttentionBias):
    """:2564-2603: ``softcap * tanh(scores / softcap)``; grad ``1 - tanh^2``."""

    def __init__(self, softcap: float = 20.0):
        if softcap <= 0:
            raise ValueError("softcap must be > 0")
        self.softcap = float(softcap)

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        c = np.asarray(self.softcap, dtype=np.asarray(scores).dtype)
        return c * np.tanh(scores / c)

    def grad(self, scores, h_idx=None, q_idx=None, k_idx=None, data=None):
        c = np.asarray(self.softcap, dtype=np.asarray(scores).dtype)
        t = np.tanh(scores / c)
        return 1.0 - t * t

    def grad_tile(self, scores, b, h, q0, bq, k0, kc):
        return self.grad(scores)


class PerHeadScaleBias(AttentionBias):
    """:2606-2648: ``scores * scales[h|0]``; grad ``scales[h|0]``."""

    def __init__(self, scales):
        s = np.asarray(scales, dtype=np.float32)
        if s.ndim == 0:
            s = s[None]
        if s.ndim != 1:
            raise ValueError("scales must be shape [H|1]")
        self.scales = s

    def _scale(self, h):
        return self.scales[0 if self.scales.shape[0] == 1 else int(h)]

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        return scores * np.asarray(self._scale(h_idx), dtype=np.asarray(scores).dtype)

    def grad_tile(self, scores, b, h, q0, bq, k0, kc):
        # The modifier's derivative at head h (the XLA path's autodiff).
        return np.full_like(scores, self._scale(h))


class LowRankBias(AttentionBias):
    """:1926-2024: ``scores + scale * U[h, q] . V[h, k]``, factors
    ``[H|1, max_length, rank]``."""

    def __init__(self, query_factors, key_factors, *, scale: float = 1.0):
        qf = np.asarray(query_factors, np.float32)
        kf = np.asarray(key_factors, np.float32)
        if qf.ndim == 2:
            qf = qf[None]
        if kf.ndim == 2:
            kf = kf[None]
        if qf.ndim != 3 or kf.ndim != 3 or qf.shape[-1] != kf.shape[-1] or qf.shape[0] != kf.shape[0]:
            raise ValueError("factors must have shape [H|1, length, rank] with one rank and head count")
        if scale < 0:
            raise ValueError("scale must be non-negative")
        self.query_factors, self.key_factors, self.scale = qf, kf, float(scale)

    @property
    def rank(self):
        return self.query_factors.shape[-1]

    def factors(self, q_len, kv_len, num_heads):
        """:1962-1995 -> ``[1, length, heads, rank]``."""
        if self.query_factors.shape[0] not in (1, num_heads):
            raise ValueError("factor head count cannot broadcast")
        qf = np.broadcast_to(self.query_factors[:, :q_len], (num_heads, q_len, self.rank))
        kf = np.broadcast_to(self.key_factors[:, :kv_len], (num_heads, kv_len, self.rank))
        return np.swapaxes(qf, 0, 1)[None], np.swapaxes(kf, 0, 1)[None]

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        # :1997-2013
        head = 0 if self.query_factors.shape[0] == 1 else int(h_idx)
        u = self.query_factors[head][np.asarray(q_idx)]
        v = self.key_factors[head][np.asarray(k_idx)]
        return scores + np.float32(self.scale) * (u @ v.T)


class BatchedLowRankBias(AttentionBias):
    """:2028-2190: per-example ``scale * U[b, q] . V[b, k]`` (factors
    ``[B, length, rank]``, a query length of 1 broadcasting); evaluated per
    example as ``dense`` (:2154-2180) does."""

    def __init__(self, query_factors, key_factors, *, scale: float = 1.0):
        qf = np.asarray(query_factors, np.float32)
        kf = np.asarray(key_factors, np.float32)
        if qf.ndim != 3 or kf.ndim != 3 or qf.shape[-1] != kf.shape[-1] or qf.shape[0] != kf.shape[0]:
            raise ValueError("factors must have shape [B, length, rank] with one rank and batch")
        if scale < 0:
            raise ValueError("scale must be non-negative")
        self.query_factors, self.key_factors, self.scale = qf, kf, float(scale)

    @classmethod
    def from_key_bias(cls, key_bias, q_len=1):
        kb = np.asarray(key_bias, np.float32)
        return cls(np.ones((kb.shape[0], q_len, 1), np.float32), kb[..., None])

    @property
    def rank(self):
        return self.query_factors.shape[-1]

    def factors(self, q_len, kv_len, num_heads):
        """:2089-2124 -> ``[B, length, heads, rank]``."""
        b = self.query_factors.shape[0]
        qf = self.query_factors if self.query_factors.shape[1] == 1 else self.query_factors[:, :q_len]
        qf = np.broadcast_to(qf[:, :, None, :], (b, q_len, num_heads, self.rank))
        kf = np.broadcast_to(self.key_factors[:, :kv_len, None, :], (b, kv_len, num_heads, self.rank))
        return qf, kf

    def tile_add(self, scores, b, h, q0, bq, k0, kc):
        qf = self.query_factors[b]
        u = np.broadcast_to(qf, (bq, self.rank)) if qf.shape[0] == 1 else qf[q0 : q0 + bq]
        v = self.key_factors[b, k0 : k0 + kc]
        return scores + np.float32(self.scale) * (u @ v.T)


class LearnedAlibiBias(AttentionBias):
    """:2258-2352: ``scores - slopes[h] * ((q + q_off) - (k + k_off))``, as
    the rank-2 factors ``U = [-s q_pos, 1]``, ``V = [1, s k_pos]``."""

    rank = 2
    scale = 1.0

    def __init__(self, slopes, *, query_offset=0, key_offset=0):
        sl = np.asarray(slopes, np.float32)
        if sl.ndim == 0:
            sl = sl[None]
        if sl.ndim != 1:
            raise ValueError("slopes must have shape [H|1]")
        self.slopes, self.query_offset, self.key_offset = sl, int(query_offset), int(key_offset)

    def factors(self, q_len, kv_len, num_heads):
        """:2291-2318 -> ``[1, length, heads, 2]``."""
        sl = np.broadcast_to(self.slopes, (num_heads,))
        qp = np.arange(q_len, dtype=np.float32) + self.query_offset
        kp = np.arange(kv_len, dtype=np.float32) + self.key_offset
        qf = np.stack((-sl[:, None] * qp[None], np.ones((num_heads, q_len), np.float32)), -1)
        kf = np.stack((np.ones((num_heads, kv_len), np.float32), sl[:, None] * kp[None]), -1)
        return np.swapaxes(qf, 0, 1)[None], np.swapaxes(kf, 0, 1)[None]

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        # :2320-2334
        head = 0 if self.slopes.shape[0] == 1 else int(h_idx)
        qp = np.asarray(q_idx) + self.query_offset
        kp = np.asarray(k_idx) + self.key_offset
        return scores - self.slopes[head] * (qp[:, None] - kp[None, :]).astype(np.float32)


def relative_position_bucket(relative_position, *, num_buckets, max_distance, bidirectional):
    """T5 bucketing of ``k - q`` (attention_mask_bias.py:2417-2449)."""
    rp = -np.asarray(relative_position, np.int64)
    if bidirectional:
        half = num_buckets // 2
        sign_bucket = (rp < 0).astype(np.int64) * half
        rp = np.abs(rp)
        nb = half
    else:
        sign_bucket = 0
        rp = np.maximum(rp, 0)
        nb = num_buckets
    max_exact = nb // 2
    small = rp < max_exact
    rpf = rp.astype(np.float32)
    large = np.float32(max_exact) + (
        np.log(np.maximum(rpf, np.float32(1.0)) / np.float32(max_exact))
        / np.log(np.float32(max_distance) / np.float32(max_exact))
        * np.float32(nb - max_exact)
    ).astype(np.float32)
    large = np.minimum(nb - 1, large.astype(np.int64))
    return np.where(small, rp, large) + sign_bucket


class T5RelativePositionBias(AttentionBias):
    """:2453-2517: ``scores + table[h|0, bucket(k - q)]``."""

    def __init__(self, bias_table, *, num_buckets, max_distance=128, bidirectional=True):
        bt = np.asarray(bias_table, np.float32)
        if bt.ndim == 1:
            bt = bt[None]
        if bt.ndim != 2 or bt.shape[-1] != num_buckets:
            raise ValueError("bias_table must have shape [H|1, num_buckets]")
        self.bias_table, self.num_buckets = bt, int(num_buckets)
        self.max_distance, self.bidirectional = int(max_distance), bool(bidirectional)

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        rel = np.asarray(k_idx)[None, :] - np.asarray(q_idx)[:, None]
        bk = relative_position_bucket(rel, num_buckets=self.num_buckets, max_distance=self.max_distance,
                                      bidirectional=self.bidirectional)
        row = self.bias_table[0 if self.bias_table.shape[0] == 1 else int(h_idx)]
        return scores + row[bk]


class LearnedRelativePositionBias(AttentionBias):
    """:2521-2561: ``scores + table[h|0, clip(k - q, -d, d) + d]``."""

    def __init__(self, table, *, max_distance):
        t = np.asarray(table, np.float32)
        if t.ndim == 1:
            t = t[None]
        if t.ndim != 2 or t.shape[-1] != 2 * int(max_distance) + 1:
            raise ValueError("table must have shape [H|1, 2*max_distance+1]")
        self.table, self.max_distance = t, int(max_distance)

    def __call__(self, scores, h_idx, q_idx, k_idx, data=None):
        rel = np.asarray(k_idx)[None, :] - np.asarray(q_idx)[:, None]
        rel = np.clip(rel, -self.max_distance, self.max_distance) + self.max_distance
        row = self.table[0 if self.table.shape[0] == 1 else int(h_idx)]
        return scores + row[rel]


class SumBias(AttentionBias):
    def __init__(self, lhs: AttentionBias, rhs: AttentionBias):
        self.lhs, self.rhs = lhs, rhs

    def tile_add(self, scores, b, h, q0, bq, k0, kc):
        # attention_mask_bias.py:563-570: scores + (s1 - s) + (s2 - s)
        s1 = self.lhs.tile_add(scores, b, h, q0, bq, k0, kc)
        s2 = self.rhs.tile_add(scores, b, h, q0, bq, k0, kc)
        return scores + (s1 - scores) + (s2 - scores)
