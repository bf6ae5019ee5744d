"""numpy restatement of probjax's XLA attention reference (the oracle).

Follows ``probjax/nn/pallas_kernels/kernels/attention_xla.py``:

* ``auto_strategy``      -- ``:586-592`` (dense <= 256^2 scores, single tile
  <= 512^2, else 256 x 256 tiles); ``_balanced_block`` ``:595-598``
* ``xla_attention``      -- ``:601-721`` (layout ``[B, T, H, D]``, GQA query
  head ``h`` -> KV head ``h // (Hq // Hkv)`` via ``[B, Hkv, G, Q, D]``,
  zero-padding to whole tiles ``:663-675``, output cast to q's dtype ``:677-679``)
* ``_scores`` / ``_pv``  -- ``:339-350`` (fp32 scores times ``sm_scale``; P cast
  to V's dtype before the P.V product, fp32 accumulation)
* ``_apply_mods``        -- ``_Mods.apply`` ``:227-279`` (bias first, then the
  mask, masked scores -> ``-inf``; padded keys masked ``:269-271``)
* ``_dense_forward``     -- ``:353-366`` (non-finite row max -> 0; ``l == 0`` -> 1;
  P normalised before the cast)
* ``_tiled_forward``     -- ``:380-429`` (online softmax; statically empty tiles
  skipped ``:318-331,373-377``; empty rows -> output 0, LSE ``+inf``)

bf16 / fp16 inputs are float32 arrays holding bfloat16 / float16 values with
``dtype="bf16"`` / ``"f16"``: products are exact in fp32, P and the output are
rounded like the reference's ``astype(bfloat16)`` / ``astype(float16)`` casts.  Dropout is off the path (rate 0) and not restated.

Parity pinned (``tests/test_oracle_attention.py``) by: float64 brute force on
tiny inputs; torch ``scaled_dot_product_attention`` on CPU (an independent
library, with ``is_causal``/boolean ``attn_mask``/``enable_gqa``); GQA ==
``np.repeat`` K/V (reference ``tests/test_attention_xla.py:379-405``); fully
masked rows exactly 0 (``:241-258``); dense == tiled for every tile size;
bf16 within 2e-2 of fp32 (``:408-421``); the LSE against ``scipy``'s
``logsumexp`` (reference ``tests/test_attention_gqa_splitkv.py:190-201``).
"""

from __future__ import annotations

import math

import numpy as np

from .bf16 import LOW_PRECISION, round_to

DENSE_MAX_SCORES = 256 * 256
SINGLE_TILE_MAX_SCORES = 512 * 512
DEFAULT_BLOCK_Q = 256
DEFAULT_BLOCK_K = 256


def auto_strategy(q_len: int, kv_len: int):
    """``(strategy, block_q, block_k)`` (attention_xla.py:586-592)."""
    if q_len * kv_len <= DENSE_MAX_SCORES:
        return "dense", None, None
    if q_len * kv_len <= SINGLE_TILE_MAX_SCORES:
        return "tiled", q_len, kv_len
    return "tiled", DEFAULT_BLOCK_Q, DEFAULT_BLOCK_K


def balanced_block(length: int, target: int) -> int:
    """attention_xla.py:595-598."""
    n = max(1, math.ceil(length / target))
    return math.ceil(length / n)


class _Mods:
    """Bias + mask evaluation on a ``[B, Hq, bq, kc]`` score tile."""

    def __init__(self, mask, bias, q_len, kv_len, kv_pad):
        self.mask, self.bias = mask, bias
        self.kv_len = kv_len
        self.kv_padded = kv_pad != kv_len

    @property
    def active(self):
        return self.mask is not None or self.bias is not None or self.kv_padded

    def apply(self, s, q0, bq, k0, kc):
        """attention_xla.py:227-279: bias, then mask; masked -> -inf."""
        if not self.active:
            return s
        B, H = s.shape[:2]
        span_q = q0 + np.arange(bq, dtype=np.int32)
        span_k = k0 + np.arange(kc, dtype=np.int32)
        if self.bias is not None:
            s = np.stack(
                [
                    np.stack(
                        [self.bias.tile_add(s[b, h], b, h, q0, bq, k0, kc) for h in range(H)]
                    )
                    for b in range(B)
                ]
            ).astype(s.dtype, copy=False)
        keep = None
        if self.mask is not None:
            keep = np.stack([self.mask.tile_keep(b, span_q, span_k) for b in range(B)])
            keep = keep[:, None]
        if self.kv_padded:
            valid = (span_k < self.kv_len)[None, None, None, :]
            keep = valid if keep is None else keep & valid
        if keep is not None:
            s = np.where(keep, s, -np.inf).astype(s.dtype, copy=False)
        return s


def _scores(q5, kc, sm_scale, cdt):
    """attention_xla.py:339-344: einsum('bhgqd,bhkd->bhgqk') * sm_scale."""
    s = np.matmul(q5.astype(cdt), np.swapaxes(kc, -1, -2).astype(cdt)[:, :, None])
    if sm_scale != 1.0:
        s = s * cdt(sm_scale)
    b, hkv, g, q, k = s.shape
    return s.reshape(b, hkv * g, q, k)


def _pv(p, vc, hkv, dtype, cdt):
    """attention_xla.py:347-350: P cast to V's dtype, fp32 accumulation."""
    b, hq, q, k = p.shape
    p5 = p.reshape(b, hkv, hq // hkv, q, k)
    if dtype in LOW_PRECISION:
        p5 = round_to(p5, dtype)
    return np.matmul(p5.astype(cdt), vc.astype(cdt)[:, :, None])


def _dense_forward(q5, k, v, mods, sm_scale, dtype, cdt):
    """attention_xla.py:353-366."""
    hkv = k.shape[1]
    q_len, kv_len = q5.shape[3], k.shape[2]
    s = mods.apply(_scores(q5, k, sm_scale, cdt), 0, q_len, 0, kv_len)
    m = np.max(s, axis=-1)
    m = np.where(np.isfinite(m), m, cdt(0.0))
    with np.errstate(invalid="ignore"):
        p = np.exp(s - m[..., None])
    l_ = np.sum(p, axis=-1)
    nonempty = l_ > 0
    lse = np.where(nonempty, m + np.log(np.where(nonempty, l_, 1.0)), np.inf)
    l_ = np.where(l_ == 0.0, cdt(1.0), l_)
    p = p / l_[..., None]
    return _pv(p, v, hkv, dtype, cdt), lse


def _tiled_forward(q5, k, v, mods, sm_scale, bq, kc, bm, dtype, cdt):
    """attention_xla.py:380-429: online softmax over bq x kc tiles."""
    b, hkv, g, q_total, _ = q5.shape
    dv = v.shape[-1]
    hq = hkv * g
    nq, nk = q_total // bq, k.shape[2] // kc
    o_out = np.zeros((b, hkv, g, q_total, dv), cdt)
    lse_out = np.zeros((b, hq, q_total), cdt)
    for i in range(nq):
        q0 = i * bq
        qi = q5[:, :, :, q0 : q0 + bq]
        o = np.zeros((b, hkv, g, bq, dv), cdt)
        m = np.full((b, hq, bq), -np.inf, cdt)
        l_ = np.zeros((b, hq, bq), cdt)
        for j in range(nk):
            if bm is not None and not bm[i, j]:
                continue  # statically fully masked tile (lax.cond skip)
            k0 = j * kc
            kj, vj = k[:, :, k0 : k0 + kc], v[:, :, k0 : k0 + kc]
            s = mods.apply(_scores(qi, kj, sm_scale, cdt), q0, bq, k0, kc)
            m_new = np.maximum(m, np.max(s, axis=-1))
            m_safe = np.where(np.isfinite(m_new), m_new, cdt(0.0))
            corr = np.exp(m - m_safe)
            p = np.exp(s - m_safe[..., None])
            l_ = l_ * corr + np.sum(p, axis=-1)
            corr5 = corr.reshape(b, hkv, g, bq)[..., None]
            o = o * corr5 + _pv(p, vj, hkv, dtype, cdt)
            m = m_new
        nonempty = l_ > 0.0
        l_safe = np.where(nonempty, l_, cdt(1.0))
        o_out[:, :, :, q0 : q0 + bq] = o / l_safe.reshape(b, hkv, g, bq)[..., None]
        lse_out[:, :, q0 : q0 + bq] = np.where(nonempty, m + np.log(l_safe), np.inf)
    return o_out, lse_out


def _tile_block_mask(mask, q_total, kv_total, bq, kc):
    """attention_xla.py:318-331."""
    if mask is None:
        return None
    bm = mask.block_mask(q_total, kv_total, bq, kc)
    if bm is None:
        return None
    bm = np.asarray(bm, dtype=bool)
    if bm.shape != (q_total // bq, kv_total // kc) or bm.all():
        return None
    return bm


def xla_attention(
    q,
    k,
    v,
    mask=None,
    bias=None,
    sm_scale: float = 1.0,
    strategy: str = "auto",
    block_q: int | None = None,
    block_k: int | None = None,
    dtype: str = "f32",
    compute_dtype=np.float32,
    return_lse: bool = False,
):
    """Oracle of ``xla_attention`` (attention_xla.py:601-721).

    ``q [B, Lq, Hq, D]``, ``k/v [B, Lk, Hkv, D|Dv]`` numpy arrays.  ``dtype``
    is the input dtype being emulated (``"f32"``, ``"bf16"`` or ``"f16"``).
    Returns the output ``[B, Lq, Hq, Dv]`` (float32; rounded to the 16-bit
    dtype for ``"bf16"`` / ``"f16"``)
    and, with ``return_lse``, the natural-log LSE ``[B, Hq, Lq]`` (``+inf``
    for rows with no valid key).
    """
    cdt = np.dtype(compute_dtype).type
    q, k, v = (round_to(np.asarray(x, np.float32), dtype) for x in (q, k, v))
    batch, q_len, hq, _ = q.shape
    kv_len, hkv = k.shape[1], k.shape[2]
    if hq % hkv != 0:
        raise ValueError(f"query heads {hq} must be a multiple of kv heads {hkv}")
    if v.shape[:3] != k.shape[:3]:
        raise ValueError(f"k {k.shape} and v {v.shape} must agree on [B, T, H]")
    g = hq // hkv

    if strategy == "auto":
        strategy, abq, abk = auto_strategy(q_len, kv_len)
        block_q, block_k = block_q or abq, block_k or abk
    if strategy == "dense":
        bq, kc = q_len, kv_len
    elif strategy == "tiled":
        bq = balanced_block(q_len, block_q or DEFAULT_BLOCK_Q)
        kc = balanced_block(kv_len, block_k or DEFAULT_BLOCK_K)
    else:
        raise ValueError(f"unknown strategy {strategy!r}")
    q_pad = math.ceil(q_len / bq) * bq
    kv_pad = math.ceil(kv_len / kc) * kc

    def to_bhtd(x, total):
        x = np.transpose(x, (0, 2, 1, 3))
        if x.shape[2] != total:
            x = np.pad(x, [(0, 0), (0, 0), (0, total - x.shape[2]), (0, 0)])
        return np.ascontiguousarray(x)

    q5 = to_bhtd(q, q_pad).reshape(batch, hkv, g, q_pad, q.shape[-1])
    kt, vt = to_bhtd(k, kv_pad), to_bhtd(v, kv_pad)
    mods = _Mods(mask, bias, q_len, kv_len, kv_pad)

    if strategy == "dense":
        o5, lse = _dense_forward(q5, kt, vt, mods, sm_scale, dtype, cdt)
    else:
        bm = _tile_block_mask(mask, q_pad, kv_pad, bq, kc)
        o5, lse = _tiled_forward(q5, kt, vt, mods, sm_scale, bq, kc, bm, dtype, cdt)

    o = o5.reshape(batch, hq, q_pad, v.shape[-1])[:, :, :q_len]
    o = np.transpose(o, (0, 2, 1, 3)).astype(np.float32)
    o = round_to(o, dtype)
    if return_lse:
        return o, np.asarray(lse[:, :, :q_len], np.float32)
    return o
