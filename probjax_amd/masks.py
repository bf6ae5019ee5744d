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
* ``ComposeMask``     -- :324-525; only ``"and"`` compositions lower to the
  kernels (what the kernels evaluate is an AND of the above);
* ``DenseBias``       -- :1807-1922, ``scores + bias[b|0, h|0, q, k]`` with an
  fp32 ``[B|1, H|1, Q, K]`` tensor.

The kernels evaluate these in-kernel: ``lower_mask`` / ``lower_bias`` turn an
object into the kernel's arguments (``causal``, per-batch ``kv_lengths``,
static ``q_valid``/``kv_valid``, the bias tensor) and return ``None`` for
anything the kernels cannot compute exactly, so that a route can fall
through.  Objects from probjax itself are recognised by class name and
fields, so the route can also be handed probjax's own mask objects.
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
    """Base class of additive score biases."""


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


class DenseBias(AttentionBias):
    def __init__(self, bias):
        if bias.ndim != 4:
            raise ValueError("bias must have shape [B|1, H|1, Q, K]")
        self.bias = bias


def _name(obj) -> str:
    return type(obj).__name__


def _is_stateful(m) -> bool:
    return _name(m) == "KVLenMask" or (
        _name(m) == "ComposeMask" and (_is_stateful(m.lhs) or _is_stateful(m.rhs))
    )


@dataclass
class LoweredMask:
    """Kernel arguments of a mask: AND of causal, per-batch KV length and
    static query / key lengths."""

    causal: bool = False
    kv_lengths: object = None  # [B] int lengths (tensor, array or sequence) or None
    q_valid: int | None = None
    kv_valid: int | None = None

    def merge(self, other: "LoweredMask") -> "LoweredMask | None":
        if self.kv_lengths is not None and other.kv_lengths is not None:
            return None  # two stateful masks: not representable (and refused by ComposeMask)
        qv = [v for v in (self.q_valid, other.q_valid) if v is not None]
        kv = [v for v in (self.kv_valid, other.kv_valid) if v is not None]
        return LoweredMask(
            causal=self.causal or other.causal,
            kv_lengths=self.kv_lengths if self.kv_lengths is not None else other.kv_lengths,
            q_valid=min(qv) if qv else None,
            kv_valid=min(kv) if kv else None,
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
        return LoweredMask(causal=True)
    if name == "KVLenMask":
        return LoweredMask(kv_lengths=mask.kv_lengths)
    if name == "QKVLengthMask":
        return LoweredMask(q_valid=int(mask.q_length), kv_valid=int(mask.kv_length))
    if name == "ComposeMask" and getattr(mask, "op", None) == "and":
        lhs, rhs = lower_mask(mask.lhs), lower_mask(mask.rhs)
        if lhs is None or rhs is None:
            return None
        return lhs.merge(rhs)
    return None


def lower_bias(bias):
    """The dense fp32 bias tensor of ``bias`` (``None`` for no bias), or the
    sentinel ``False`` when the kernels cannot add it exactly."""
    if bias is None:
        return None
    if _name(bias) == "DenseBias":
        b = bias.bias
        return b if isinstance(b, torch.Tensor) else torch.as_tensor(b)
    return False
