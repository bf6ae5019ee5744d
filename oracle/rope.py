"""Rotary position encoding, restated (oracle).

Follows ``probjax/nn/layers/encoding.py``: ``inv_freq_i = base^(-2i/d)``
(``:171-175``), angles ``pos * inv_freq`` (``:177-190``), and the interleaved
even/odd pair rotation ``(x0, x1) -> (x0 cos - x1 sin, x1 cos + x0 sin)``
(``:204-211``).

Parity pinned (``tests/test_oracle_latent.py``): the rotation preserves norms,
``<R(m) q, R(n) k>`` depends only on ``m - n``, position 0 is the identity, and
``inv_freq`` matches its closed form at ``i = 0`` and ``i = d/2 - 1``.
"""

import numpy as np


def inv_freq(rotary_dim: int, base: float = 10000.0, dtype=np.float32):
    """encoding.py:171-175."""
    exponents = np.arange(0, rotary_dim, 2, dtype=dtype) / dtype(rotary_dim)
    return (1.0 / (dtype(base) ** exponents)).astype(dtype)


def cos_sin(positions, freqs):
    """encoding.py:177-190."""
    angles = np.asarray(positions, freqs.dtype)[:, None] * freqs[None, :]
    return np.cos(angles), np.sin(angles)


def apply_rotary(x, positions, base: float = 10000.0):
    """Rotate the last axis of ``x [..., T, (H,) d]`` at ``positions [T]``.

    ``x`` is ``[..., T, d]`` or ``[..., T, H, d]``; angles broadcast over H.
    """
    x = np.asarray(x, np.float32)
    d = x.shape[-1]
    cos, sin = cos_sin(positions, inv_freq(d, base))
    if x.ndim >= 3 and x.shape[-3] == len(positions):  # [..., T, H, d]
        cos, sin = cos[:, None, :], sin[:, None, :]
    even, odd = x[..., ::2], x[..., 1::2]
    r_even = even * cos - odd * sin
    r_odd = odd * cos + even * sin
    return np.stack((r_even, r_odd), axis=-1).reshape(x.shape).astype(np.float32)
