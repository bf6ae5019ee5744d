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

import torch


class AttentionMask:
    """Base class: ``mask & other`` composes with a logical AND."""

    def __and__(self, other):
        return ComposeMask("and", self, other)

    def __or__(self, other):
        return ComposeMask("or", self, other)

    def __xor__(self, other):
        return ComposeMask("xor", self, other)


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

    @property
    def extended(self) -> bool:
        return (self.alibi is not None or self.softcap > 0 or self.head_scales is not None
                or self.constant != 0.0)


_ADDITIVE = ("DenseBias", "IdentityBias", "ConstantBias", "CausalAlibiBias", "SymmetricAlibiBias",
             "DistanceDecayBias")


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
            if lb.dense is not None:
                return False
            b = p.bias
            lb.dense = b if isinstance(b, torch.Tensor) else torch.as_tensor(b)
        elif pn == "ConstantBias":
            lb.constant += float(p.value)
        elif pn in ("CausalAlibiBias", "SymmetricAlibiBias", "DistanceDecayBias"):
            if lb.alibi is not None:
                return False
            lb.alibi = {"CausalAlibiBias": "causal", "SymmetricAlibiBias": "symmetric",
                        "DistanceDecayBias": "decay"}[pn]
            lb.alibi_alpha = float(getattr(p, "alpha", 1.0))
    return lb
