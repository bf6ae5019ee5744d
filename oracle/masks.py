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
* ``SumBias``        -- ``:551-577`` (sum of additive deltas)

The XLA reference evaluates a mask per ``(batch, head)`` on index tiles with
its payload sliced per batch (``attention_xla.py:227-279``); ``tile_keep``
below is that evaluation for one batch element, ``tile_add`` the bias one.

Parity pinned by the reference's own known-answer tests, restated in
``tests/test_oracle_masks.py`` (``tests/test_attention_mask_bias.py:54-68,
130-163, 263-294`` in the reference) and by the equivalence
KVLenMask(L) == boolean key mask ``arange(S) < L`` == additive -inf bias.
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
        raise NotImplementedError  # pragma: no cover


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


class SumBias(AttentionBias):
    def __init__(self, lhs: AttentionBias, rhs: AttentionBias):
        self.lhs, self.rhs = lhs, rhs

    def tile_add(self, scores, b, h, q0, bq, k0, kc):
        # attention_mask_bias.py:563-570: scores + (s1 - s) + (s2 - s)
        s1 = self.lhs.tile_add(scores, b, h, q0, bq, k0, kc)
        s2 = self.rhs.tile_add(scores, b, h, q0, bq, k0, kc)
        return scores + (s1 - scores) + (s2 - scores)
