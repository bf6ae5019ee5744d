"""Mask and bias objects of the fused-attention path, lowered to kernel arguments.

Same names, constructor arguments and semantics as probjax's mask/bias pytrees
for the objects this path supports (probjax/nn/pallas_kernels/
attention_mask_bias.py):

* ``NoMask``          -- :583-612, every key kept;
* ``CausalMask``      -- :615-646, key ``k`` kept for query ``q`` iff ``q >= k``
  (top-left aligned);
* ``QKVLengthMask``   -- :1077-1127, static ``(q < q_length) & (k < kv_length)``;
* ``KVLenMask``       -- :1399-1532, key ``k`` of batch ``b`` kept iff
  ``k < kv_lengths[b]``;
* ``CausalFromBottomRightMask`` -- :753-782, ``q + (kv_length - q_length) >= k``;
* ``LocalWindowMask`` / ``CausalLocalWindowMask`` -- :651-750, a band
  ``q - left <= k <= q + right`` (right 0 for the causal one);
* ``PrefixLMMask``    -- :785-868, ``k < P[b]`` or ``q >= k``;
* ``SeqLenMask``      -- :1239-1398, full attention inside ``L[b]``, the
  diagonal outside;
* ``SameSegmentMask`` / ``BlockDiagonalMask`` / ``BlockDiagonalCausalMask`` --
  :1537-1668, :871-1076, equal segment ids (and ``q >= k``);
* ``KeyPaddingMask``  -- :1132-1236, key ``k`` kept for query row ``q`` iff
  ``k < key_lengths`` read per query row (the reference's payload layout:
  ``[T]`` gives row ``i`` the count ``kl[i]`` in every batch, ``[B, T]``
  gives ``kl[b, i]``, rows past ``T`` count 0, a scalar holds everywhere);
* ``ComposeMask``     -- :324-525; only ``"and"`` compositions lower to the
  kernels (what the kernels evaluate is an AND of the above);
* ``DenseBias``       -- :1807-1922, ``scores + bias[b|0, h|0, q, k]`` with an
  fp32 ``[B|1, H|1, Q, K]`` tensor;
* ``NotMask`` / OR / XOR compositions / ``MarginalizationMask`` (:530-548,
  :324-525, :1671-1778) and ``T5RelativePositionBias`` /
  ``LearnedRelativePositionBias`` (:2417-2561) -- no in-kernel form: the
  route lowers them to a dense additive bias (``dense_keep``,
  ``dense_relpos``);
* low-rank biases     -- ``LowRankBias``, ``BatchedLowRankBias``,
  ``LearnedAlibiBias`` (:1926-2352): ``flex_attention`` and
  ``dot_product_attention`` fold their factors into Q/K
  (``split_low_rank_bias``), as probjax's ``flex_attention`` does;
* score modifiers     -- ``IdentityBias``, ``ConstantBias``, ``CausalAlibiBias``,
  ``SymmetricAlibiBias``, ``DistanceDecayBias`` (additive, composable with
  ``+`` / ``SumBias`` :553-582) and ``SoftCappingBias`` / ``PerHeadScaleBias``
  (alone: the reference's SumBias gives every child the derivative 1,
  :286-298).

The kernels evaluate these in-kernel: ``lower_mask`` / ``lower_bias`` turn an
object into the kernel's arguments (``causal`` and its shift, per-batch
``kv_lengths``, static ``q_valid``/``kv_valid``, window bounds, per-batch
prefix / sequence lengths, segment ids, the bias tensor, the modifiers) and
return ``None`` / ``False`` for anything the kernels cannot compute exactly,
so that a route can fall through.  Objects from probjax itself are
recognised by class name and fields, so the route can also be handed
probjax's own mask objects.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


class AttentionMask:
    """Base class: ``mask & other`` composes with a logical AND."""

    def __and__(self, other):
        return ComposeMask("and", self, other)

    def __or__(self, other):
        return ComposeMask("or", self, other)

    def __xor__(self, other):
        return ComposeMask("xor", self, other)

    def __invert__(self):
        return NotMask(self)


class AttentionBias:
    """Base class of score biases; ``a + b`` composes (SumBias)."""

    def __add__(self, other):
        return SumBias(self, other)


class NoMask(AttentionMask):
    pass


class CausalMask(AttentionMask):
    pass


class QKVLengthMask(AttentionMask):
    def __init__(self, q_length: int, kv_length: int, block_sparse: bool = True):
        self.q_length = int(q_length)
        self.kv_length = int(kv_length)
        self.block_sparse = block_sparse


class KVLenMask(AttentionMask):
    def __init__(self, kv_lengths):
        self.kv_lengths = kv_lengths


class ComposeMask(AttentionMask):
    def __init__(self, op: str, lhs: AttentionMask, rhs: AttentionMask):
        if op not in ("and", "or", "xor"):
            raise ValueError(f"Unknown op for ComposeMask: {op}")
        if _is_stateful(lhs) and _is_stateful(rhs):
            raise ValueError("Cannot compose two stateful masks")
        self.op, self.lhs, self.rhs = op, lhs, rhs


class CausalFromBottomRightMask(AttentionMask):
    def __init__(self, q_length: int, kv_length: int):
        self.q_length, self.kv_length = int(q_length), int(kv_length)


class LocalWindowMask(AttentionMask):
    def __init__(self, left_window: int, right_window: int | None = None):
        self.left_window = int(left_window)
        self.right_window = right_window


class CausalLocalWindowMask(AttentionMask):
    def __init__(self, left_window: int):
        self.left_window = int(left_window)


class PrefixLMMask(AttentionMask):
    def __init__(self, prefix_lengths):
        self.prefix_lengths = prefix_lengths


class SeqLenMask(AttentionMask):
    def __init__(self, seq_lengths):
        self.seq_lengths = seq_lengths


class SameSegmentMask(AttentionMask):
    def __init__(self, query_segment_ids, key_segment_ids=None):
        self.query_segment_ids = query_segment_ids
        self.key_segment_ids = key_segment_ids


class BlockDiagonalMask(AttentionMask):
    def __init__(self, query_block_ids, key_block_ids=None):
        self.query_block_ids = query_block_ids
        self.key_block_ids = key_block_ids


class BlockDiagonalCausalMask(BlockDiagonalMask):
    pass


class KeyPaddingMask(AttentionMask):
    def __init__(self, key_lengths):
        self.key_lengths = key_lengths


class NotMask(AttentionMask):
    def __init__(self, inner):
        self.inner = inner


class MarginalizationMask(AttentionMask):
    def __init__(self, mask):
        self.mask = mask


class DenseBias(AttentionBias):
    def __init__(self, bias):
        if bias.ndim != 4:
            raise ValueError("bias must have shape [B|1, H|1, Q, K]")
        self.bias = bias


class SumBias(AttentionBias):
    def __init__(self, lhs: AttentionBias, rhs: AttentionBias):
        self.lhs, self.rhs = lhs, rhs


class IdentityBias(AttentionBias):
    pass


class ConstantBias(AttentionBias):
    def __init__(self, value: float):
        self.value = float(value)


class CausalAlibiBias(AttentionBias):
    pass


class SymmetricAlibiBias(AttentionBias):
    pass


class DistanceDecayBias(AttentionBias):
    def __init__(self, alpha: float = 1.0):
        self.alpha = float(alpha)


class SoftCappingBias(AttentionBias):
    def __init__(self, softcap: float = 20.0):
        if softcap <= 0:
            raise ValueError("softcap must be > 0")
        self.softcap = float(softcap)


class PerHeadScaleBias(AttentionBias):
    def __init__(self, scales):
        self.scales = scales


class T5RelativePositionBias(AttentionBias):
    """``scores + table[h|0, bucket(k - q)]`` (attention_mask_bias.py:2453-2517)."""

    def __init__(self, bias_table, *, num_buckets: int, max_distance: int = 128, bidirectional: bool = True):
        bt = torch.as_tensor(bias_table)
        if bt.ndim == 1:
            bt = bt[None]
        if bt.ndim != 2:
            raise ValueError("bias_table must have shape [H|1, num_buckets]")
        if int(bt.shape[-1]) != int(num_buckets):
            raise ValueError("bias_table last dim must equal num_buckets")
        self.bias_table, self.num_buckets = bt, int(num_buckets)
        self.max_distance, self.bidirectional = int(max_distance), bool(bidirectional)


class LearnedRelativePositionBias(AttentionBias):
    """``scores + table[h|0, clip(k - q, -d, d) + d]`` (attention_mask_bias.py:2521-2561)."""

    def __init__(self, table, *, max_distance: int):
        t = torch.as_tensor(table)
        if t.ndim == 1:
            t = t[None]
        if t.ndim != 2:
            raise ValueError("table must have shape [H|1, 2*max_distance+1]")
        if int(t.shape[-1]) != 2 * int(max_distance) + 1:
            raise ValueError("table last dim must be 2*max_distance+1")
        self.table, self.max_distance = t, int(max_distance)


class LowRankBias(AttentionBias):
    """``scale * U[h, q] . V[h, k]`` with factors ``[H|1, max_length, rank]``
    (attention_mask_bias.py:1926-2024); ``flex_attention`` folds the factors
    into Q/K."""

    def __init__(self, query_factors, key_factors, *, scale: float = 1.0):
        qf, kf = torch.as_tensor(query_factors), torch.as_tensor(key_factors)
        if qf.ndim == 2:
            qf = qf[None]
        if kf.ndim == 2:
            kf = kf[None]
        if qf.ndim != 3 or kf.ndim != 3:
            raise ValueError("factors must have shape [H|1, length, rank]")
        if qf.shape[-1] != kf.shape[-1]:
            raise ValueError("query and key factors must have the same rank")
        if qf.shape[0] != kf.shape[0]:
            raise ValueError("query and key factors must have the same head count")
        if scale < 0:
            raise ValueError("scale must be non-negative")
        self.query_factors, self.key_factors, self.scale = qf, kf, float(scale)

    @property
    def rank(self) -> int:
        return self.query_factors.shape[-1]

    def factors(self, q_len: int, kv_len: int, num_heads: int, *, dtype=None):
        """Factors in attention layout ``[1, length, heads, rank]`` (:1962-1995)."""
        if q_len > self.query_factors.shape[1]:
            raise ValueError(f"q_len={q_len} exceeds maximum {self.query_factors.shape[1]}")
        if kv_len > self.key_factors.shape[1]:
            raise ValueError(f"kv_len={kv_len} exceeds maximum {self.key_factors.shape[1]}")
        fh = self.query_factors.shape[0]
        if fh not in (1, num_heads):
            raise ValueError(f"factor head count {fh} cannot broadcast to {num_heads}")
        qf = self.query_factors[:, :q_len].expand(num_heads, q_len, self.rank)
        kf = self.key_factors[:, :kv_len].expand(num_heads, kv_len, self.rank)
        qf, kf = qf.transpose(0, 1)[None], kf.transpose(0, 1)[None]
        if dtype is not None:
            qf, kf = qf.to(dtype), kf.to(dtype)
        return qf, kf


class BatchedLowRankBias(AttentionBias):
    """Per-example ``scale * U[b, q] . V[b, k]`` with factors ``[B, length,
    rank]`` (a query length of 1 broadcasts; attention_mask_bias.py:2028-2190)."""

    def __init__(self, query_factors, key_factors, *, scale: float = 1.0):
        qf, kf = torch.as_tensor(query_factors), torch.as_tensor(key_factors)
        if qf.ndim != 3 or kf.ndim != 3:
            raise ValueError("factors must have shape [B, length, rank]")
        if qf.shape[-1] != kf.shape[-1]:
            raise ValueError("query and key factors must have the same rank")
        if qf.shape[0] != kf.shape[0]:
            raise ValueError("query and key factors must have the same batch size")
        if scale < 0:
            raise ValueError("scale must be non-negative")
        self.query_factors, self.key_factors, self.scale = qf, kf, float(scale)

    @classmethod
    def from_key_bias(cls, key_bias, q_len: int = 1):
        """Rank-1 bias adding ``key_bias[b, k]`` to every score of key ``k`` (:2069-2083)."""
        kb = torch.as_tensor(key_bias)
        if kb.ndim != 2:
            raise ValueError("key_bias must have shape [B, kv_len]")
        ones = torch.ones((kb.shape[0], q_len, 1), dtype=kb.dtype, device=kb.device)
        return cls(ones, kb[..., None])

    @property
    def rank(self) -> int:
        return self.query_factors.shape[-1]

    def factors(self, q_len: int, kv_len: int, num_heads: int, *, dtype=None):
        """Factors in attention layout ``[B, length, heads, rank]`` (:2089-2124)."""
        b = self.query_factors.shape[0]
        if self.query_factors.shape[1] == 1:
            qf = self.query_factors[:, :, None, :]
        elif q_len <= self.query_factors.shape[1]:
            qf = self.query_factors[:, :q_len, None, :]
        else:
            raise ValueError(f"q_len={q_len} exceeds maximum {self.query_factors.shape[1]}")
        if kv_len > self.key_factors.shape[1]:
            raise ValueError(f"kv_len={kv_len} exceeds maximum {self.key_factors.shape[1]}")
        kf = self.key_factors[:, :kv_len, None, :]
        qf = qf.expand(b, q_len, num_heads, self.rank)
        kf = kf.expand(b, kv_len, num_heads, self.rank)
        if dtype is not None:
            qf, kf = qf.to(dtype), kf.to(dtype)
        return qf, kf


class LearnedAlibiBias(AttentionBias):
    """``-slopes[h] * ((q + query_offset) - (k + key_offset))`` as a rank-2
    factorisation, so gradients reach ``slopes`` (attention_mask_bias.py:
    2258-2352)."""

    def __init__(self, slopes, *, query_offset: int = 0, key_offset: int = 0):
        sl = torch.as_tensor(slopes)
        if sl.ndim == 0:
            sl = sl[None]
        if sl.ndim != 1:
            raise ValueError("slopes must have shape [H|1]")
        self.slopes, self.query_offset, self.key_offset = sl, int(query_offset), int(key_offset)

    rank = 2
    scale = 1.0

    def factors(self, q_len: int, kv_len: int, num_heads: int, *, dtype=None):
        """``U = [-s * q_pos, 1]``, ``V = [1, s * k_pos]`` in layout
        ``[1, length, heads, 2]`` (:2291-2318)."""
        if self.slopes.shape[0] not in (1, num_heads):
            raise ValueError(f"slope head count {self.slopes.shape[0]} cannot broadcast to {num_heads}")
        sl = self.slopes.expand(num_heads)
        qp = torch.arange(q_len, dtype=sl.dtype, device=sl.device) + self.query_offset
        kp = torch.arange(kv_len, dtype=sl.dtype, device=sl.device) + self.key_offset
        qf = torch.stack((-sl[:, None] * qp[None], torch.ones(num_heads, q_len, dtype=sl.dtype, device=sl.device)), -1)
        kf = torch.stack((torch.ones(num_heads, kv_len, dtype=sl.dtype, device=sl.device), sl[:, None] * kp[None]), -1)
        qf, kf = qf.transpose(0, 1)[None], kf.transpose(0, 1)[None]
        if dtype is not None:
            qf, kf = qf.to(dtype), kf.to(dtype)
        return qf, kf


_LOW_RANK = ("LowRankBias", "BatchedLowRankBias", "LearnedAlibiBias")


def split_low_rank_bias(bias):
    """``(low-rank terms, remaining bias)`` (probjax ``_split_low_rank_bias``,
    layers/attention.py:1322-1345): the terms ``flex_attention`` folds into
    Q/K, out of a bias or a ``SumBias`` tree."""
    if bias is None:
        return [], None
    name = _name(bias)
    if name in _LOW_RANK:
        return [bias], None
    if name == "SumBias":
        lt, lhs = split_low_rank_bias(bias.lhs)
        rt, rhs = split_low_rank_bias(bias.rhs)
        rest = rhs if lhs is None else lhs if rhs is None else SumBias(lhs, rhs)
        return lt + rt, rest
    return [], bias


def _name(obj) -> str:
    return type(obj).__name__


_STATEFUL = ("KVLenMask", "PrefixLMMask", "SeqLenMask", "SameSegmentMask", "BlockDiagonalMask",
             "BlockDiagonalCausalMask", "KeyPaddingMask")


def _is_stateful(m) -> bool:
    return _name(m) in _STATEFUL or (
        _name(m) == "ComposeMask" and (_is_stateful(m.lhs) or _is_stateful(m.rhs))
    )


def _min_opt(a, b):
    vals = [v for v in (a, b) if v is not None]
    return min(vals) if vals else None


@dataclass
class LoweredMask:
    """Kernel arguments of a mask: an AND of positional intervals (causal with
    a shift, a window), per-batch KV / prefix / sequence lengths, segment ids
    and static query / key lengths."""

    causal_shift: int | None = None  # None: no causal bound; 0: CausalMask
    kv_lengths: object = None  # [B] int lengths (tensor, array or sequence) or None
    q_valid: int | None = None
    kv_valid: int | None = None
    window_left: int | None = None
    window_right: int | None = None
    prefix_lengths: object = None  # scalar or [B]
    seq_lengths: object = None  # [B]
    segment_q: object = None  # [B, Lq] or [Lq]
    segment_k: object = None  # [B, Lk] or [Lk] (None: the query ids)
    row_kv_lengths: object = None  # KeyPaddingMask payload: scalar, [T] or [B, T]

    @property
    def causal(self) -> bool:
        return self.causal_shift is not None

    @property
    def extended(self) -> bool:
        """Needs the kernels' extended-mask path (anything beyond causal,
        KV lengths and static lengths)."""
        return (
            (self.causal_shift not in (None, 0))
            or self.window_left is not None
            or self.window_right is not None
            or self.prefix_lengths is not None
            or self.seq_lengths is not None
            or self.segment_q is not None
            or self.row_kv_lengths is not None
        )

    def merge(self, other: "LoweredMask") -> "LoweredMask | None":
        state = [
            n for n in ("kv_lengths", "prefix_lengths", "seq_lengths", "segment_q", "row_kv_lengths")
            for m in (self, other) if getattr(m, n) is not None
        ]
        if len(state) > 1:
            return None  # two stateful masks: not representable (and refused by ComposeMask)
        pick = lambda n: getattr(self, n) if getattr(self, n) is not None else getattr(other, n)  # noqa: E731
        return LoweredMask(
            causal_shift=_min_opt(self.causal_shift, other.causal_shift),
            kv_lengths=pick("kv_lengths"),
            q_valid=_min_opt(self.q_valid, other.q_valid),
            kv_valid=_min_opt(self.kv_valid, other.kv_valid),
            window_left=_min_opt(self.window_left, other.window_left),
            window_right=_min_opt(self.window_right, other.window_right),
            prefix_lengths=pick("prefix_lengths"),
            seq_lengths=pick("seq_lengths"),
            segment_q=pick("segment_q"),
            segment_k=pick("segment_k"),
            row_kv_lengths=pick("row_kv_lengths"),
        )


def lower_mask(mask) -> LoweredMask | None:
    """Kernel arguments for ``mask``, or ``None`` if the kernels cannot
    evaluate it exactly (any other mask type, an OR / XOR composition)."""
    if mask is None:
        return LoweredMask()
    name = _name(mask)
    if name == "NoMask":
        return LoweredMask()
    if name == "CausalMask":
        return LoweredMask(causal_shift=0)
    if name == "CausalFromBottomRightMask":
        return LoweredMask(causal_shift=int(mask.kv_length) - int(mask.q_length))
    if name == "LocalWindowMask":
        rw = 0 if mask.right_window is None else int(mask.right_window)
        if mask.left_window < 0 or rw < 0:
            return None
        return LoweredMask(window_left=int(mask.left_window), window_right=rw)
    if name == "CausalLocalWindowMask":
        if mask.left_window < 0:
            return None
        return LoweredMask(window_left=int(mask.left_window), window_right=0)
    if name == "KVLenMask":
        return LoweredMask(kv_lengths=mask.kv_lengths)
    if name == "PrefixLMMask":
        return LoweredMask(prefix_lengths=mask.prefix_lengths)
    if name == "SeqLenMask":
        return LoweredMask(seq_lengths=mask.seq_lengths)
    if name == "SameSegmentMask":
        return LoweredMask(segment_q=mask.query_segment_ids, segment_k=mask.key_segment_ids)
    if name in ("BlockDiagonalMask", "BlockDiagonalCausalMask"):
        return LoweredMask(segment_q=mask.query_block_ids, segment_k=mask.key_block_ids,
                           causal_shift=0 if name == "BlockDiagonalCausalMask" else None)
    if name == "KeyPaddingMask":
        return LoweredMask(row_kv_lengths=mask.key_lengths)
    if name == "QKVLengthMask":
        return LoweredMask(q_valid=int(mask.q_length), kv_valid=int(mask.kv_length))
    if name == "ComposeMask" and getattr(mask, "op", None) == "and":
        lhs, rhs = lower_mask(mask.lhs), lower_mask(mask.rhs)
        if lhs is None or rhs is None:
            return None
        return lhs.merge(rhs)
    return None


@dataclass
class LoweredBias:
    """Kernel arguments of a bias: s' = f(s) + dense + alibi + constant with
    f the soft cap, the per-head scale or the identity."""

    dense: object = None  # [B|1, H|1, Q, K] tensor
    alibi: str | None = None  # "causal" (2^-(h+1), relu), "symmetric" (2^-(h+1), |.|), "decay"
    alibi_alpha: float = 1.0  # DistanceDecayBias
    softcap: float = 0.0
    head_scales: object = None  # [H|1]
    constant: float = 0.0
    relpos: list = None  # T5 / learned relative-position terms, added to ``dense`` per call
    distance: list = None  # further (kind, alpha) distance terms past the first, added to ``dense`` per call
    dense_more: list = None  # further DenseBias tensors, added to ``dense`` per call

    @property
    def extended(self) -> bool:
        return (self.alibi is not None or self.softcap > 0 or self.head_scales is not None
                or self.constant != 0.0)


_ADDITIVE = ("DenseBias", "IdentityBias", "ConstantBias", "CausalAlibiBias", "SymmetricAlibiBias",
             "DistanceDecayBias", "T5RelativePositionBias", "LearnedRelativePositionBias")


def _flatten_sum(bias, out) -> bool:
    name = _name(bias)
    if name == "SumBias":
        return _flatten_sum(bias.lhs, out) and _flatten_sum(bias.rhs, out)
    if name not in _ADDITIVE:
        return False
    out.append(bias)
    return True


def lower_bias(bias):
    """Kernel arguments of ``bias`` (``None`` for no bias), or the sentinel
    ``False`` when the kernels cannot apply it exactly."""
    if bias is None:
        return None
    name = _name(bias)
    if name == "SoftCappingBias":
        return LoweredBias(softcap=float(bias.softcap))
    if name == "PerHeadScaleBias":
        sc = bias.scales
        return LoweredBias(head_scales=sc if isinstance(sc, torch.Tensor) else torch.as_tensor(sc))
    parts = []
    if not _flatten_sum(bias, parts):
        return False
    lb = LoweredBias()
    for p in parts:
        pn = _name(p)
        if pn == "DenseBias":
            b = p.bias
            b = b if isinstance(b, torch.Tensor) else torch.as_tensor(b)
            if lb.dense is None:
                lb.dense = b
            else:  # a sum of dense terms: one tensor (SumBias, attention_mask_bias.py:551-577)
                lb.dense_more = (lb.dense_more or []) + [b]
        elif pn == "ConstantBias":
            lb.constant += float(p.value)
        elif pn in ("T5RelativePositionBias", "LearnedRelativePositionBias"):
            lb.relpos = (lb.relpos or []) + [p]
        elif pn in ("CausalAlibiBias", "SymmetricAlibiBias", "DistanceDecayBias"):
            kind = {"CausalAlibiBias": "causal", "SymmetricAlibiBias": "symmetric",
                    "DistanceDecayBias": "decay"}[pn]
            alpha = float(getattr(p, "alpha", 1.0))
            if lb.alibi is None:
                lb.alibi, lb.alibi_alpha = kind, alpha
            else:  # the kernels evaluate one distance term; further ones go dense
                lb.distance = (lb.distance or []) + [(kind, alpha)]
    return lb


# ---------------------------------------------------------------------------
# Dense forms, for the masks and biases without an in-kernel form (NOT / OR /
# XOR compositions, MarginalizationMask, relative-position tables): the
# kernels take them as an additive fp32 bias (0 / -inf for a mask), which is
# exact and costs Lq * Lk floats per (batch, head) slice.
# ---------------------------------------------------------------------------

def _per_position(payload, B, n, device, dtype):
    """A ``[T]`` (every batch) or ``[B, T]`` payload read at positions
    ``0..n-1``, zero past ``T`` (how the reference's XLA path windows a
    per-position payload, attention_xla.py:130-133, 146-168); None when the
    batch does not match."""
    t = torch.as_tensor(payload, device=device)
    if t.ndim == 1:
        t = t[None].expand(B, -1)
    elif t.ndim != 2 or t.shape[0] != B:
        return None
    out = torch.zeros((B, n), dtype=dtype, device=device)
    m = min(int(t.shape[1]), n)
    out[:, :m] = t[:, :m].to(dtype)
    return out


def _per_batch(x, B, device):
    t = torch.as_tensor(x, device=device).reshape(-1)
    if t.numel() == 1:
        t = t.expand(B)
    return t if t.numel() == B else None


def dense_keep(mask, B, l_q, l_k, device):
    """``[B, Lq, Lk]`` boolean keep-mask of any mask object of the path
    (attention_mask_bias.py semantics, stateful payloads read as the XLA path
    reads them), or None when a payload does not fit the call."""
    q = torch.arange(l_q, device=device)[None, :, None]
    k = torch.arange(l_k, device=device)[None, None, :]
    if mask is None:
        return torch.ones((B, l_q, l_k), dtype=torch.bool, device=device)
    name = _name(mask)

    def full(x):
        return x.expand(B, l_q, l_k)

    if name == "NoMask":
        return full(torch.ones((1, 1, 1), dtype=torch.bool, device=device))
    if name == "CausalMask":
        return full(k <= q)
    if name == "CausalFromBottomRightMask":
        return full(k <= q + (int(mask.kv_length) - int(mask.q_length)))
    if name == "LocalWindowMask":
        rw = 0 if mask.right_window is None else int(mask.right_window)
        return full((k >= q - int(mask.left_window)) & (k <= q + rw))
    if name == "CausalLocalWindowMask":
        return full((k >= q - int(mask.left_window)) & (k <= q))
    if name == "QKVLengthMask":
        return full((q < int(mask.q_length)) & (k < int(mask.kv_length)))
    if name in ("KVLenMask", "PrefixLMMask", "SeqLenMask"):
        attr = {"KVLenMask": "kv_lengths", "PrefixLMMask": "prefix_lengths", "SeqLenMask": "seq_lengths"}[name]
        L = _per_batch(getattr(mask, attr), B, device)
        if L is None:
            return None
        L = L.to(torch.int64)[:, None, None]
        if name == "KVLenMask":
            return full(k < L)
        if name == "PrefixLMMask":
            return (k < L) | (k <= q)
        return ((q < L) & (k < L)) | (q == k)
    if name in ("SameSegmentMask", "BlockDiagonalMask", "BlockDiagonalCausalMask"):
        qa = "query_segment_ids" if name == "SameSegmentMask" else "query_block_ids"
        ka = "key_segment_ids" if name == "SameSegmentMask" else "key_block_ids"
        kid = getattr(mask, ka) if getattr(mask, ka) is not None else getattr(mask, qa)
        sq = torch.as_tensor(getattr(mask, qa), device=device)
        sk = torch.as_tensor(kid, device=device)
        if sq.shape[-1] != l_q or sk.shape[-1] != l_k:
            return None
        sq = sq.reshape(-1, l_q).expand(B, -1) if sq.ndim == 1 or sq.shape[0] == 1 else sq
        sk = sk.reshape(-1, l_k).expand(B, -1) if sk.ndim == 1 or sk.shape[0] == 1 else sk
        if sq.shape[0] != B or sk.shape[0] != B:
            return None
        keep = sq[:, :, None] == sk[:, None, :]
        return keep & (k <= q) if name == "BlockDiagonalCausalMask" else keep
    if name == "KeyPaddingMask":
        kl = torch.as_tensor(mask.key_lengths, device=device)
        if kl.dtype.is_floating_point:
            return None
        rows = (kl.to(torch.int64).reshape(1, 1).expand(B, l_q) if kl.ndim == 0
                else _per_position(kl.to(torch.int64), B, l_q, device, torch.int64))
        return None if rows is None else k < rows[:, :, None]
    if name == "MarginalizationMask":
        mq = _per_position(mask.mask, B, l_q, device, torch.bool)
        mk = _per_position(mask.mask, B, l_k, device, torch.bool)
        if mq is None or mk is None:
            return None
        return (mq[:, :, None] & mk[:, None, :]) | (q == k)
    if name == "NotMask":
        inner = dense_keep(mask.inner, B, l_q, l_k, device)
        return None if inner is None else ~inner
    if name == "ComposeMask":
        lhs = dense_keep(mask.lhs, B, l_q, l_k, device)
        rhs = dense_keep(mask.rhs, B, l_q, l_k, device)
        if lhs is None or rhs is None:
            return None
        return {"and": torch.logical_and, "or": torch.logical_or, "xor": torch.logical_xor}[mask.op](lhs, rhs)
    return None


_DENSE_MASKS = ("NoMask", "CausalMask", "CausalFromBottomRightMask", "LocalWindowMask", "CausalLocalWindowMask",
                "QKVLengthMask", "KVLenMask", "PrefixLMMask", "SeqLenMask", "SameSegmentMask", "BlockDiagonalMask",
                "BlockDiagonalCausalMask", "KeyPaddingMask", "MarginalizationMask")


def dense_supported(mask) -> bool:
    """Whether ``dense_keep`` knows every node of ``mask``."""
    if mask is None:
        return True
    name = _name(mask)
    if name == "NotMask":
        return dense_supported(mask.inner)
    if name == "ComposeMask":
        return getattr(mask, "op", None) in ("and", "or", "xor") and dense_supported(mask.lhs) and dense_supported(mask.rhs)
    return name in _DENSE_MASKS


def _t5_bucket_lut(rel, num_buckets, max_distance, bidirectional):
    """T5 buckets of ``k - q`` values ``rel`` (attention_mask_bias.py:
    2417-2449), float32 arithmetic as the reference."""
    rp = -rel.astype(np.int64)
    if bidirectional:
        half = num_buckets // 2
        sign = (rp < 0).astype(np.int64) * half
        rp = np.abs(rp)
        nb = half
    else:
        sign = 0
        rp = np.maximum(rp, 0)
        nb = num_buckets
    max_exact = nb // 2
    large = np.float32(max_exact) + (
        np.log(np.maximum(rp.astype(np.float32), np.float32(1.0)) / np.float32(max_exact))
        / np.log(np.float32(max_distance) / np.float32(max_exact)) * np.float32(nb - max_exact)
    ).astype(np.float32)
    large = np.minimum(nb - 1, large.astype(np.int64))
    return np.where(rp < max_exact, rp, large) + sign


def dense_distance(kind, alpha, h_q, l_q, l_k, device):
    """``[1, H|1, Lq, Lk]`` fp32 values of a distance bias: CausalAlibiBias
    ``-2^-(h+1) * relu(q - k)`` (attention_mask_bias.py:2223-2255),
    SymmetricAlibiBias ``-2^-(h+1) * |q - k|`` (:2355-2380) or
    DistanceDecayBias ``-alpha * |q - k|`` (:2387-2414)."""
    d = (torch.arange(l_q, device=device)[:, None] - torch.arange(l_k, device=device)[None, :]).to(torch.float32)
    f = d.clamp_min(0.0) if kind == "causal" else d.abs()
    if kind == "decay":
        return (-float(alpha) * f)[None, None]
    slopes = torch.pow(2.0, -(torch.arange(h_q, device=device, dtype=torch.float32) + 1.0))
    return -(slopes[:, None, None] * f[None])[None]


def dense_relpos(term, l_q, l_k, device):
    """``[1, H|1, Lq, Lk]`` fp32 values of a T5 / learned relative-position
    term; differentiable in its table (a gather)."""
    rel_vals = np.arange(-(l_q - 1), l_k, dtype=np.int64)  # every k - q
    if _name(term) == "T5RelativePositionBias":
        lut = _t5_bucket_lut(rel_vals, term.num_buckets, term.max_distance, term.bidirectional)
        table = term.bias_table
    else:
        d = term.max_distance
        lut = np.clip(rel_vals, -d, d) + d
        table = term.table
    lut_t = torch.as_tensor(lut, device=device)
    idx = lut_t[torch.arange(l_k, device=device)[None, :] - torch.arange(l_q, device=device)[:, None] + (l_q - 1)]
    return table.to(device=device, dtype=torch.float32)[:, idx][None]
