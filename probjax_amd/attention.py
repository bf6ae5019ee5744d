"""probjax.nn's fused-attention API served by the MI355X (gfx950) HIP kernels.

The functions keep probjax's names, argument meanings, defaults and error
messages for the fused-attention path, on torch tensors resident on a ROCm
device (torch provides the HBM buffers and the stream; the arithmetic is the
HIP library behind ``include/probjax_hip.h``):

* ``hip_attention_or_none`` -- a route with the protocol of probjax's
  ``cudnn_attention_or_none`` / ``mosaic_attention_or_none``
  (probjax/nn/layers/attention_device.py:165-237): inputs ``[B, T, H, D]``,
  returns the output, or ``None`` to fall through; ``force=True`` skips the
  device table and the environment switch;
* ``flex_attention`` / ``dot_product_attention`` -- the dispatchers
  (layers/attention.py:1205-1319, 1426-1759) with ``implementation="hip"``
  (or ``None`` = the device table) in place of the Triton/cuDNN/Mosaic
  choices; default ``sm_scale = 1/sqrt(D)``;
* ``mha`` -- the kernel API (pallas_kernels/kernels/attention.py:2692-2984),
  default ``sm_scale = 1.0``, split-KV decoding chosen by ``use_splitkv``
  (:2653-2689) extended to ``KVLenMask``;
* gradients -- when q, k or v requires grad, the flash path (and the split-KV
  primal) runs as a ``torch.autograd.Function`` whose backward is the HIP
  backward (probjax's custom VJP of ``mha``, :3188-3266; no cotangent for
  mask/bias data);
* ``splitkv_forward`` -- kernels/attention_splitkv.py:137-250;
* ``mla`` -- kernels/latent_attention.py:636-766, absorbed form (``wk = wv =
  None``), default ``sm_scale = 1/sqrt(qk_head_dim)``.

There is no CPU or library fallback: a call the kernels cannot compute
exactly raises ``ValueError`` (forced paths) or returns ``None`` (the route),
and a missing kernel library raises ``NativeLibraryError``.

Device table: the route is on by default on gfx950 devices; set
``PROBJAX_ATTENTION_HIP=0`` to turn the default route off (forced calls still
run), mirroring ``PROBJAX_ATTENTION_CUDNN`` / ``PROBJAX_ATTENTION_MOSAIC``.
"""

from __future__ import annotations

import functools
import math
import os

import torch

from . import hip_attention as hip
from .masks import (LoweredBias, LoweredMask, dense_distance, dense_keep, dense_relpos, dense_supported, lower_bias,
                    lower_mask, split_low_rank_bias)

HIP_ARCH = "gfx950"
HALF_DTYPES = (torch.bfloat16, torch.float16)  # the 16-bit (MFMA bf16 / fp16) kernels
KERNEL_DTYPES = HALF_DTYPES + (torch.float32,)  # dtypes the kernels take
FLASH_HEAD_DIMS = (64, 128, 256)
FLASH_HEAD_DIMS_F32 = (64, 128, 256)
DECODE_HEAD_DIMS = (64, 128, 256)  # head dims (q/k and v each) of the split-KV decode
LATENT_WIDTHS = (512, 576)  # latent ranks of the wide absorbed-mla kernels (16-bit)
# Lq*H folded rows up to which an absorbed decode step takes the split-KV latent
# kernel: each 16 rows form a row group that streams the cache, so up to 8
# passes over it; longer query blocks run the latent flash kernels, whose
# 128-row query tiles read it once per tile.
MLA_DECODE_MAX_ROWS = 128
MLA_SHAPES = ((576, 512), (576, 576), (512, 512), (256, 256), (128, 128), (64, 64))  # (rank, v_dim)


def _mla_decode_shape(rank: int, v_dim: int):
    """The latent decode kernel's (rank, v_dim) that carries a latent of width
    ``rank`` and the first ``v_dim`` output columns: the narrowest rank >= rank
    (zero-padded: zero features change no score), then the narrowest output
    width >= v_dim (the extra columns are sliced off); None when too wide."""
    fits = [(r, d) for r, d in MLA_SHAPES if r >= rank and d >= v_dim]
    return min(fits) if fits else None
BACKWARD_DTYPES = KERNEL_DTYPES  # dtypes pjx_flash_bwd takes

# Split-KV decode thresholds (probjax kernels/attention.py:2649-2650).
_SPLITKV_MAX_Q_LEN = 64
_SPLITKV_MIN_KV_LEN = 1024


def _env_off(name: str) -> bool:
    """attention_device.py:67-68."""
    return os.environ.get(name, "1").strip().lower() in ("0", "false", "no", "off")


@functools.lru_cache(maxsize=None)
def _device_arch(index: int) -> str:
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def hip_device(t) -> bool:
    """``t`` lives on a gfx950 ROCm device."""
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        return False
    return _device_arch(t.device.index if t.device.index is not None else 0) == HIP_ARCH


def device_table_enabled() -> bool:
    return not _env_off("PROBJAX_ATTENTION_HIP") and not _env_off("PROBJAX_ATTENTION_DEVICE_DEFAULTS")


# ---------------------------------------------------------------------------
# Eligibility
# ---------------------------------------------------------------------------

def _lengths_tensor(kv_lengths, batch, device):
    L = torch.as_tensor(kv_lengths, device=device).reshape(-1)
    if L.numel() != batch:
        return None
    return L.to(torch.int32)


def _row_kv_lengths(kl, B, l_q, device):
    """``[B, Lq]`` int32 key count of every query row of a ``KeyPaddingMask``
    payload, or None.

    The reference reads the payload per query position (its ``get_data`` and
    query block spec, attention_mask_bias.py:1175-1204, windowed by
    attention_xla.py:130-133, 146-168): a vector ``[T]`` gives row ``i`` the
    count ``kl[i]`` in every batch, ``[B, T]`` gives ``kl[b, i]``, rows past
    ``T`` read the zero fill, a scalar holds for every row; the mask then
    keeps ``k < count`` (:1143-1164, a boolean payload comparing as 0/1).
    """
    t = torch.as_tensor(kl, device=device)
    if t.dtype.is_floating_point or t.dtype.is_complex:
        return None
    t = t.to(torch.int32)
    if t.ndim == 0:
        return t.reshape(1, 1).expand(B, l_q).contiguous()
    if t.ndim == 1:
        t = t[None].expand(B, -1)
    elif t.ndim != 2 or t.shape[0] != B:
        return None
    out = torch.zeros((B, l_q), dtype=torch.int32, device=device)
    n = min(int(t.shape[1]), l_q)
    out[:, :n] = t[:, :n]
    return out


def _decode_plan(query, key, value, lm: LoweredMask, lb: LoweredBias | None):
    """Arguments of the split-KV decode for this call, or None."""
    if lb is not None or lm.causal or lm.extended or lm.q_valid is not None or lm.kv_valid is not None:
        return None
    if query.dtype not in KERNEL_DTYPES:
        return None
    if query.shape[-1] not in DECODE_HEAD_DIMS or value.shape[-1] not in DECODE_HEAD_DIMS:
        return None
    return dict(kv_lengths=lm.kv_lengths)


def _int_tensor(x, shape, device):
    """int32 device tensor of ``x`` broadcast to ``shape``, or None."""
    t = torch.as_tensor(x, device=device)
    if t.dtype.is_floating_point or t.dtype == torch.bool:
        return None
    try:
        return torch.broadcast_to(t.to(torch.int32), shape).contiguous()
    except RuntimeError:
        return None


def _score_mods(lm: LoweredMask, lb: LoweredBias | None, B, l_q, l_k, h_q, device):
    """``ScoreModsArgs`` of the extended masks / modifiers (None when there
    are none), or False when their data does not fit the call."""
    ext_bias = lb is not None and lb.extended
    if not lm.extended and not ext_bias:
        return None
    m = hip.ScoreModsArgs(causal_shift=lm.causal_shift or 0)
    if lm.window_left is not None:
        m.window_left = int(lm.window_left)
    if lm.window_right is not None:
        m.window_right = int(lm.window_right)
    for name, val in (("prefix_lengths", lm.prefix_lengths), ("seq_lengths", lm.seq_lengths)):
        if val is not None:
            t = _int_tensor(torch.as_tensor(val).reshape(-1), (B,), device)
            if t is None:
                return False
            setattr(m, name, t)
    if lm.row_kv_lengths is not None:
        m.row_kv_lengths = lm.row_kv_lengths  # [B, Lq] int32 (prepared by _eligible)
    if lm.segment_q is not None:
        kid = lm.segment_k if lm.segment_k is not None else lm.segment_q
        sq, sk = torch.as_tensor(lm.segment_q), torch.as_tensor(kid)
        if sq.shape[-1] != l_q or sk.shape[-1] != l_k:
            return False  # ids per position (keys default to the query ids)
        m.segment_q = _int_tensor(sq, (B, l_q), device)
        m.segment_k = _int_tensor(sk, (B, l_k), device)
        if m.segment_q is None or m.segment_k is None:
            return False
    if lb is not None:
        if lb.alibi is not None:
            if lb.alibi == "decay":
                slopes = torch.full((h_q,), lb.alibi_alpha, dtype=torch.float32)
            else:
                slopes = torch.tensor([2.0 ** (-(h + 1.0)) for h in range(h_q)], dtype=torch.float32)
            m.alibi_slopes = slopes.to(device)
            m.alibi_symmetric = lb.alibi != "causal"
        m.softcap = float(lb.softcap)
        m.constant = float(lb.constant)
        if lb.head_scales is not None:
            hs = torch.as_tensor(lb.head_scales, dtype=torch.float32).reshape(-1)
            if hs.numel() not in (1, h_q):
                return False
            m.head_scales = torch.broadcast_to(hs, (h_q,)).contiguous().to(device)
    return m


def _flash_plan(query, key, value, lm: LoweredMask, lb: LoweredBias | None, check_dim: bool = True):
    """Arguments of the flash forward for this call, or None (``check_dim``:
    the head dim must be a flash kernel width)."""
    if query.dtype not in KERNEL_DTYPES:
        return None
    B, l_q, h_q, d = query.shape
    l_k = key.shape[1]
    if check_dim and _kernel_width(d, query.dtype) != d:
        return None
    dense = None if lb is None else lb.dense
    if dense is not None:
        if dense.ndim != 4 or tuple(dense.shape[-2:]) != (l_q, l_k):
            return None
        if dense.shape[0] not in (1, B) or dense.shape[1] not in (1, h_q):
            return None
    mods = _score_mods(lm, lb, B, l_q, l_k, h_q, query.device)
    if mods is False:
        return None
    return dict(causal=lm.causal, kv_lengths=lm.kv_lengths, bias=dense,
                q_valid=lm.q_valid, kv_valid=lm.kv_valid, mods=mods)


def _eligible(query, key, value, *, mask, bias, dropout_rate):
    """(lowered mask, bias tensor) when the kernels compute the call exactly."""
    if dropout_rate > 0.0:
        return None
    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        return None
    if not (query.dtype == key.dtype == value.dtype):
        return None
    if not (hip_device(query) and key.device == query.device and value.device == query.device):
        return None
    B, l_q, h_q, d = query.shape
    if key.shape[0] != B or value.shape != key.shape or key.shape[-1] != d or h_q % key.shape[2]:
        return None
    lm = lower_mask(mask)
    mask_bias = None
    if lm is None:
        # no in-kernel form (NOT / OR / XOR, MarginalizationMask): an additive
        # 0 / -inf bias of the mask's dense form is exact
        keep = dense_keep(mask, B, l_q, key.shape[1], query.device)
        if keep is None:
            return None
        lm = LoweredMask()
        mask_bias = torch.zeros(keep.shape, dtype=torch.float32, device=query.device)
        mask_bias = mask_bias.masked_fill_(~keep, float("-inf"))[:, None]
    if lm.row_kv_lengths is not None:
        rows = _row_kv_lengths(lm.row_kv_lengths, B, l_q, query.device)
        if rows is None:
            return None
        if l_q == 1:
            # One query row: its count is a per-batch key length, which is what
            # MultiHeadAttention's cached decode builds each step
            # (layers/attention.py:612-675); the KV-length kernels take it.
            lm.row_kv_lengths, lm.kv_lengths = None, rows[:, 0]
        else:
            lm.row_kv_lengths = rows
    if lm.kv_lengths is not None:
        L = _lengths_tensor(lm.kv_lengths, B, query.device)
        if L is None:
            return None
        lm.kv_lengths = L
    lb = lower_bias(bias)
    if lb is False:
        return None
    if lb is not None and lb.dense is not None:
        lb.dense = lb.dense.to(device=query.device, dtype=torch.float32)
    extra = [] if mask_bias is None else [mask_bias]
    if lb is not None and lb.dense_more:
        for t in lb.dense_more:
            # each term of a dense sum must itself broadcast to [B, Hq, Lq, Lk]
            if t.ndim != 4 or tuple(t.shape[-2:]) != (l_q, key.shape[1]) or t.shape[0] not in (1, B) \
                    or t.shape[1] not in (1, h_q):
                return None
            extra.append(t.to(device=query.device, dtype=torch.float32))
        lb.dense_more = None
    if lb is not None and lb.distance:
        extra += [dense_distance(kind, alpha, h_q, l_q, key.shape[1], query.device) for kind, alpha in lb.distance]
        lb.distance = None
    if lb is not None and lb.relpos:
        for term in lb.relpos:
            rows = (term.bias_table if hasattr(term, "bias_table") else term.table).shape[0]
            if rows not in (1, h_q):
                return None
            extra.append(dense_relpos(term, l_q, key.shape[1], query.device))
        lb.relpos = None
    if extra:
        lb = lb if lb is not None else LoweredBias()
        for e in extra:
            lb.dense = e if lb.dense is None else lb.dense + e
    return lm, lb


def _splitkv_ok(q, k, lm: LoweredMask | None, has_bias: bool, dropout_rate: float,
                split_kv: bool | None) -> bool:
    if split_kv is False:
        return False
    if q.ndim != 4 or k.ndim != 4 or dropout_rate > 0 or has_bias:
        return False
    if lm is None or lm.causal or lm.extended or lm.q_valid is not None or lm.kv_valid is not None:
        return False
    if q.dtype not in KERNEL_DTYPES or _decode_width(q.shape[-1]) is None:
        return False
    if k.shape[2] <= 0 or q.shape[2] % k.shape[2]:
        return False
    if split_kv:
        return True
    return q.shape[1] <= _SPLITKV_MAX_Q_LEN and k.shape[1] >= _SPLITKV_MIN_KV_LEN


def use_splitkv(q, k, *, mask=None, bias=None, dropout_rate: float = 0.0,
                split_kv: bool | None = None) -> bool:
    """Whether ``mha`` runs the split-KV decode for these inputs.

    probjax's rule (kernels/attention.py:2653-2689): never with
    ``split_kv=False``; only exact cases (no bias, no dropout); ``True``
    forces it when exact; ``None`` picks it for ``Lq <= 64`` and
    ``Lkv >= 1024``.  The HIP decode is also exact with a ``KVLenMask`` (keys
    past each length are skipped), so a length mask does not disable it here;
    it takes bf16, fp16 and fp32, head_dim <= 256 (zero-padded to 64, 128 or
    256) and any number of packed rows ``(Hq/Hkv)*Lq`` (up to 64 per pass over
    the keys, as the reference's row blocks, attention_splitkv.py:155-172).
    """
    lm = lower_mask(mask)
    if lm is not None and lm.row_kv_lengths is not None and getattr(q, "ndim", 0) == 4 and q.shape[1] == 1:
        lm.kv_lengths, lm.row_kv_lengths = lm.row_kv_lengths, None  # one row: per-batch lengths
    return _splitkv_ok(q, k, lm, bias is not None, dropout_rate, split_kv)


class _AttentionFunction(torch.autograd.Function):
    """Differentiable HIP attention, the custom VJP of probjax's ``mha``
    (kernels/attention.py:3188-3266): the forward keeps ``(q, k, v, out,
    lse)`` as residuals and the backward is ``pjx_flash_bwd``.  Mask and bias
    data get no cotangent, as in the reference (:3262-3263), unless the dense
    bias tensor is passed as ``bias``: then it is an input and receives
    dL/d(bias) (the gradient probjax's dense ``dot_product_attention`` path,
    layers/attention.py:1293-1319, gives it)."""

    @staticmethod
    def forward(ctx, query, key, value, bias, run_fwd, bwd_kwargs):
        out, lse = run_fwd(query, key, value)
        ctx.save_for_backward(query, key, value, out, lse)
        ctx.bwd_kwargs = bwd_kwargs
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse=None):
        del dlse  # the LSE output is a residual, not differentiated
        q, k, v, o, lse = ctx.saved_tensors
        if ctx.bias_dtype is not None and ctx.needs_input_grad[3]:
            dq, dk, dv, db = hip.flash_attention_bwd(q, k, v, o, dout, lse, bias_grad=True, **ctx.bwd_kwargs)
            return dq, dk, dv, db.to(ctx.bias_dtype), None, None
        dq, dk, dv = hip.flash_attention_bwd(q, k, v, o, dout, lse, **ctx.bwd_kwargs)
        return dq, dk, dv, None, None, None


def _needs_grad(*ts) -> bool:
    return torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def _kernel_width(d: int, dtype=torch.bfloat16):
    """The flash kernels' head dim that carries head dim ``d`` in ``dtype``
    (None: too wide): 64, 128, or 256 in bfloat16 / float16."""
    widths = FLASH_HEAD_DIMS if dtype in HALF_DTYPES else FLASH_HEAD_DIMS_F32
    return next((w for w in widths if w >= d), None)


def _decode_width(d: int):
    """The split-KV decode's head dim that carries head dim ``d`` (None: too wide)."""
    return next((w for w in DECODE_HEAD_DIMS if w >= d), None)


def _pad_features(x, width):
    """``x`` with zero features appended up to ``width`` (autograd slices the
    gradient back)."""
    return torch.nn.functional.pad(x, (0, width - x.shape[-1]))


def _run(query, key, value, lm, lb, sm_scale, split_kv, bias_grad=False, want_lse=False):
    """Output of the HIP route for an eligible call (None: not computable
    exactly); with ``want_lse`` ``(output, lse [B, Hq, Lq])``, where rows
    without a valid key have ``lse = +inf``."""
    d = query.shape[-1]
    width = _kernel_width(d, query.dtype)
    if width is not None and width != d:
        # Zero features change no q.k product and add only zero output
        # columns: every kept score, weight and output element is the one the
        # width-d computation gives (the reference pads its blocks to
        # next_power_of_2(head_dim) with masked loads, kernels/attention.py:2168).
        res = _run(_pad_features(query, width), _pad_features(key, width), _pad_features(value, width),
                   lm, lb, sm_scale, split_kv, bias_grad, want_lse)
        if res is None:
            return None
        return (res[0][..., :d], res[1]) if want_lse else res[..., :d]
    dense = None if lb is None else lb.dense
    bias_in = dense if bias_grad and dense is not None and _needs_grad(dense) else None
    grad = _needs_grad(query, key, value) or bias_in is not None
    if grad and query.dtype not in BACKWARD_DTYPES:
        return None
    if _splitkv_ok(query, key, lm, lb is not None, 0.0, split_kv):
        plan = _decode_plan(query, key, value, lm, lb)
        if plan is not None:
            if not grad:
                return hip.splitkv_decode(query, key, value, sm_scale=sm_scale, return_lse=want_lse, **plan)
            # Split-KV primal, regular backward (probjax splitkv_attention,
            # kernels/attention_splitkv.py:253-272).
            res = _AttentionFunction.apply(
                query, key, value, None,
                lambda q, k, v: hip.splitkv_decode(q, k, v, sm_scale=sm_scale, return_lse=True, **plan),
                dict(sm_scale=sm_scale, kv_lengths=plan["kv_lengths"]),
            )
            return res if want_lse else res[0]
    plan = _flash_plan(query, key, value, lm, lb)
    if plan is None:
        return None
    if not grad:
        return hip.flash_attention_fwd(query, key, value, sm_scale=sm_scale, return_lse=want_lse, **plan)
    res = _AttentionFunction.apply(
        query, key, value, bias_in,
        lambda q, k, v: hip.flash_attention_fwd(q, k, v, sm_scale=sm_scale, return_lse=True, **plan),
        dict(sm_scale=sm_scale, **plan),
    )
    return res if want_lse else res[0]


# ---------------------------------------------------------------------------
# Route (selector seam)
# ---------------------------------------------------------------------------

def hip_attention_or_none(query, key, value, *, mask, bias, dropout_rate: float,
                          sm_scale: float, force: bool = False):
    """HIP fused attention when the device table routes this call there.

    Inputs are ``[B, T, H, D]`` (K/V may have fewer heads, GQA).  Returns the
    output, or None to fall through (``force=True``: skip the device table and
    the environment switch, only check that the kernels compute the call
    exactly).
    """
    if not force and not device_table_enabled():
        return None
    e = _eligible(query, key, value, mask=mask, bias=bias, dropout_rate=dropout_rate)
    if e is None:
        return None
    lm, lb = e
    return _run(query, key, value, lm, lb, float(sm_scale), None)


# ---------------------------------------------------------------------------
# Kernel API
# ---------------------------------------------------------------------------

def _gqa_group(hq: int, hkv: int) -> int:
    if hkv <= 0 or hq % hkv:
        raise ValueError(f"number of query heads ({hq}) must be a multiple of KV heads ({hkv})")
    return hq // hkv


def mha(q, k, v, mask=None, bias=None, rng=None, sm_scale: float = 1.0, *,
        dropout_rate: float = 0.0, split_kv: bool | None = None, **unused_tuning):
    """Multi-head attention (probjax ``mha``): ``q [B, Lq, Hq, D]``,
    ``k/v [B, Lk, Hkv, D]`` -> ``[B, Lq, Hq, D]``.

    ``sm_scale`` defaults to 1.0 as in probjax.  Tiling arguments of the Pallas
    API (``block_sizes``, ``num_warps``, ...) are accepted and ignored: the HIP
    kernels choose their tiles.  Raises ``ValueError`` for calls the kernels
    cannot compute exactly (dropout, masks/biases other than those in
    ``probjax_amd.masks``, unsupported dtype or head_dim).
    """
    del rng, unused_tuning
    _gqa_group(q.shape[-2], k.shape[-2])
    if v.shape[-2] != k.shape[-2]:
        raise ValueError(
            f"key and value need the same number of heads, got {k.shape[-2]} and {v.shape[-2]}."
        )
    e = _eligible(q, k, v, mask=mask, bias=bias, dropout_rate=dropout_rate)
    out = None if e is None else _run(q, k, v, e[0], e[1], float(sm_scale), split_kv)
    if out is None:
        raise ValueError(_unsupported_message(q, k, mask, bias, dropout_rate))
    return out


def _unsupported_message(q, k, mask, bias, dropout_rate) -> str:
    why = []
    if not hip_device(q):
        why.append(f"tensors must be on a {HIP_ARCH} ROCm device (got {getattr(q, 'device', None)})")
    if dropout_rate > 0:
        why.append("dropout is not supported")
    if lower_mask(mask) is None and not dense_supported(mask):
        why.append(f"mask {type(mask).__name__} is not supported")
    if lower_bias(bias) is False:
        why.append(f"bias {type(bias).__name__} is not supported")
    if getattr(q, "dtype", None) not in KERNEL_DTYPES:
        why.append(f"dtype {getattr(q, 'dtype', None)} is not supported (bf16, fp16, fp32)")
    if _needs_grad(q, k) and getattr(q, "dtype", None) not in BACKWARD_DTYPES:
        why.append(f"gradients need {BACKWARD_DTYPES} inputs (got {getattr(q, 'dtype', None)})")
    if q.ndim == 4 and _kernel_width(q.shape[-1], getattr(q, "dtype", None)) is None:
        why.append(f"head_dim {q.shape[-1]} is not supported (at most {FLASH_HEAD_DIMS[-1]} in bfloat16 / "
                   f"float16, {FLASH_HEAD_DIMS_F32[-1]} in float32)")
    detail = "; ".join(why) or "unsupported shape combination"
    return f"the HIP attention kernels cannot compute this call exactly: {detail}"


def splitkv_forward(q, k, v, *, sm_scale: float, num_splits: int | None = None,
                    block_k: int = 64, return_lse: bool = False, kv_lengths=None,
                    **unused_tuning):
    """Split-KV ("flash-decoding") forward (probjax ``splitkv_forward``,
    kernels/attention_splitkv.py:137-250): bf16 / fp16 / fp32
    ``q [B, Lq, Hq, D]``, ``k [B, Lkv, Hkv, D]``, ``v [B, Lkv, Hkv, Dv]``
    -> ``[B, Lq, Hq, Dv]``; D and Dv up to 256 (zero-padded to 64, 128 or
    256, as the reference pads its blocks to the next power of two,
    :155-172), any number of packed rows ``(Hq/Hkv)*Lq``.

    ``num_splits`` maps to KV chunks of ``ceil(Lkv / num_splits)`` keys rounded
    up to 128 (``None``: the kernel's own choice).  ``kv_lengths`` ([B]) is the
    KVLenMask extension.  With ``return_lse`` also returns the natural-log LSE
    ``[B, Hq, Lq]`` (attention_splitkv.py:248-250; ``+inf`` for empty rows).
    """
    del block_k, unused_tuning
    _gqa_group(q.shape[-2], k.shape[-2])
    d, dv = q.shape[-1], v.shape[-1]
    width, v_width = _decode_width(d), _decode_width(dv)
    if width is None or v_width is None:
        raise ValueError(f"splitkv_forward: head dims up to {DECODE_HEAD_DIMS[-1]}, got D={d}, Dv={dv}")
    if width != d:
        q, k = _pad_features(q, width), _pad_features(k, width)
    if v_width != dv:
        v = _pad_features(v, v_width)
    chunk = 0
    if num_splits is not None:
        if num_splits < 1:
            raise ValueError(f"num_splits must be >= 1, got {num_splits}")
        per = -(-k.shape[1] // num_splits)
        chunk = max(128, -(-per // 128) * 128)
    res = hip.splitkv_decode(q, k, v, sm_scale=float(sm_scale), kv_lengths=kv_lengths,
                             chunk=chunk, return_lse=return_lse)
    if v_width == dv:
        return res
    return (res[0][..., :dv], res[1]) if return_lse else res[..., :dv]


class _MaterializedMLAFunction(torch.autograd.Function):
    """Differentiable materialised latent attention: the custom VJP of
    probjax's ``mla`` with projections (latent_attention.py:527-589).

    Forward: ``pjx_mla_project`` forms ``K = C W_K^T`` and ``V = C W_V^T``
    (zero-padded to the common head width) once, then the flash forward
    attends the zero-padded ``q`` over them.  Backward: the VJP of that
    materialised computation, as in the reference (:571-589): the flash
    backward gives ``dq, dK, dV``; the projection's chain rule gives
    ``dC = dK W_K + dV W_V``, ``dW_K = dK^T C``, ``dW_V = dV^T C`` (plain
    GEMMs, the reference's einsum VJPs).  K and V are kept from the forward
    rather than formed a second time."""

    @staticmethod
    def forward(ctx, q, cache, wk, wv, st):
        o, lse = hip.flash_attention_fwd(st["qp"], st["k"], st["v"], sm_scale=st["sm_scale"],
                                         return_lse=True, **st["plan"])
        ctx.save_for_backward(cache, wk, wv, st["qp"], st["k"], st["v"], o, lse)
        ctx.st = {n: st[n] for n in ("sm_scale", "plan", "dk", "dv", "width")}
        return o if st["dv"] == st["width"] else o[..., : st["dv"]].contiguous()

    @staticmethod
    def backward(ctx, dout):
        cache, wk, wv, qp, k, v, o, lse = ctx.saved_tensors
        st = ctx.st
        dk_dim, dv_dim, width = st["dk"], st["dv"], st["width"]
        dop = _pad_head(dout.to(o.dtype), width)
        dqp, dkp, dvp = hip.flash_attention_bwd(qp, k, v, o, dop, lse, sm_scale=st["sm_scale"], **st["plan"])
        B, S, R = cache.shape
        H = wk.shape[0]
        dK = dkp[..., :dk_dim].reshape(B * S, H * dk_dim)
        dV = dvp[..., :dv_dim].reshape(B * S, H * dv_dim)
        c2 = cache.reshape(B * S, R)
        dcache = dK @ wk.reshape(H * dk_dim, R) + dV @ wv.reshape(H * dv_dim, R)
        dwk = (dK.t().contiguous() @ c2).reshape(H, dk_dim, R)
        dwv = (dV.t().contiguous() @ c2).reshape(H, dv_dim, R)
        dq = dqp if dk_dim == width else dqp[..., :dk_dim].contiguous()
        return dq, dcache.reshape(B, S, R), dwk, dwv, None


def _pad_head(x, width):
    """``x`` zero-padded on its last (head) axis to ``width`` (contiguous)."""
    if x.shape[-1] == width:
        return x.contiguous()
    out = torch.zeros(x.shape[:-1] + (width,), dtype=x.dtype, device=x.device)
    out[..., : x.shape[-1]] = x
    return out


def _mla_materialized(q, cache, wk, wv, *, mask, bias, sm_scale):
    """Materialised ``mla`` (latent_attention.py:413-468, 527-589) on the HIP
    kernels; ValueError when they cannot compute the call exactly."""
    B, l_q, H, dk_dim = q.shape
    dv_dim = wv.shape[1]
    width = _kernel_width(max(dk_dim, dv_dim), q.dtype)
    if width is None:
        top = (FLASH_HEAD_DIMS if q.dtype in HALF_DTYPES else FLASH_HEAD_DIMS_F32)[-1]
        raise ValueError(f"materialised mla supports head dims up to {top} in {q.dtype}, "
                         f"got qk {dk_dim}, v {dv_dim}")
    if not (q.dtype == cache.dtype == wk.dtype == wv.dtype) or q.dtype not in BACKWARD_DTYPES:
        raise ValueError("materialised mla takes q, cache, wk and wv of one dtype (bfloat16, float16 or float32)")
    if not all(hip_device(t) and t.device == q.device for t in (cache, wk, wv)):
        raise ValueError(f"the HIP latent-attention kernels need tensors on a {HIP_ARCH} ROCm device")
    with torch.no_grad():
        k, v = hip.mla_project(cache.detach(), wk.detach(), wv.detach(), width=width)
        qp = _pad_head(q.detach(), width)
    e = _eligible(qp, k, v, mask=mask, bias=bias, dropout_rate=0.0)
    plan = None if e is None else _flash_plan(qp, k, v, e[0], e[1])
    if plan is None:
        raise ValueError("the HIP kernels cannot compute this materialised mla call exactly: "
                         + _unsupported_message(qp, k, mask, bias, 0.0))
    st = dict(qp=qp, k=k, v=v, plan=plan, sm_scale=float(sm_scale), dk=dk_dim, dv=dv_dim, width=width)
    if not _needs_grad(q, cache, wk, wv):
        o = hip.flash_attention_fwd(qp, k, v, sm_scale=float(sm_scale), **plan)
        return o if dv_dim == width else o[..., :dv_dim]
    return _MaterializedMLAFunction.apply(q, cache, wk, wv, st)


def _absorbed_cheaper(l_q: int, kv_len: int, rank: int, dk: int, dv: int) -> bool:
    """probjax's choice between the two exact factorisations of projected
    latent attention, by FLOP count (latent_attention.py:616-620)."""
    materialized = kv_len * rank * (dk + dv) + l_q * kv_len * (dk + dv)
    absorbed = l_q * rank * (dk + dv) + 2 * l_q * kv_len * rank
    return absorbed < materialized


def _mla_absorbed_lengths(q, cache, wk, wv, mask, bias):
    """Per-batch KV lengths (or "all") when a projected ``mla`` call is cheaper
    absorbed and the latent decode kernel computes it exactly; else None."""
    B, l_q, H, dk = q.shape
    R, dv = cache.shape[-1], wv.shape[1]
    if bias is not None or _needs_grad(q, cache, wk, wv):
        return None
    if not (q.dtype == cache.dtype == wk.dtype == wv.dtype) or q.dtype not in HALF_DTYPES:
        return None
    if (R, R) not in MLA_SHAPES or l_q * H > MLA_DECODE_MAX_ROWS:
        return None
    if not _absorbed_cheaper(l_q, cache.shape[1], R, dk, dv):
        return None
    if not all(hip_device(t) and t.device == q.device for t in (q, cache, wk, wv)):
        return None
    lm = lower_mask(mask)
    if lm is None:
        return None
    if lm.row_kv_lengths is not None and l_q == 1:
        rows = _row_kv_lengths(lm.row_kv_lengths, B, 1, q.device)
        if rows is None:
            return None
        lm.row_kv_lengths, lm.kv_lengths = None, rows[:, 0]
    if lm.causal or lm.extended or lm.q_valid is not None or lm.kv_valid is not None:
        return None
    if lm.kv_lengths is None:
        return "all"
    return _lengths_tensor(lm.kv_lengths, B, q.device)


def _mla_absorbed(q, cache, wk, wv, kv_lengths, sm_scale):
    """Projected ``mla`` in the absorbed factorisation (latent_attention.py:
    621-623): ``q W_K`` attends over the latent (``K = V = C``) on the latent
    decode kernel, then ``W_V`` maps the latent-space output.  The two
    per-head products are plain batched GEMMs."""
    B, l_q, H, dk = q.shape
    R, dv = cache.shape[-1], wv.shape[1]
    qh = q.permute(2, 0, 1, 3).reshape(H, B * l_q, dk).contiguous()
    q_lat = torch.bmm(qh, wk.contiguous()).reshape(H, B, l_q, R).permute(1, 2, 0, 3).contiguous()
    o_lat = hip.mla_decode(q_lat, cache, sm_scale=float(sm_scale),
                           kv_lengths=None if isinstance(kv_lengths, str) else kv_lengths)
    oh = o_lat.permute(2, 0, 1, 3).reshape(H, B * l_q, R).contiguous()
    out = torch.bmm(oh, wv.transpose(1, 2).contiguous())
    return out.reshape(H, B, l_q, dv).permute(1, 2, 0, 3).contiguous()


def mla(q, cache, wk=None, wv=None, *, mask=None, bias=None, rng=None,
        sm_scale: float | None = None, dropout_rate: float = 0.0, v_dim: int | None = None,
        **unused_tuning):
    """Attention of ``q`` over a shared latent ``cache`` (probjax ``mla``,
    kernels/latent_attention.py:636-766).

    Absorbed form (``wk = wv = None``, ``K = V = cache``): ``q [B, Q, H, R]``,
    ``cache [B, S, R]`` -> ``[B, Q, H, R]`` (or the first ``v_dim`` columns,
    which is all a caller that multiplies by ``W_UV`` of width ``v_dim``
    needs), any query length, every mask and bias of the flash route,
    differentiable in ``q`` and ``cache`` (bias data gets no gradient, as in
    the reference's VJP); latent widths up to 576 in bfloat16 / float16 (up to 256 in
    float32).  Decode steps (``Q * H <= 128``, no gradient, no bias,
    ``None`` / ``KVLenMask``) run the split-KV latent kernel; the rest the
    latent flash kernels, whose heads share one K = V head (the folded
    ``[B, Q*H, 1, R]`` form of the reference layer is the same call with
    ``H = 1``).

    Materialised form (``wk [H, qk_head_dim, R]``, ``wv [H, v_head_dim, R]``):
    ``q [B, Q, H, qk_head_dim]`` -> ``[B, Q, H, v_head_dim]``, every mask and
    bias of the flash route (the reference's contract: equal to ``mha`` over
    the materialised K/V, tests/test_latent_attention.py:341-379), bf16 or
    fp32, differentiable in ``q``, ``cache``, ``wk`` and ``wv``; head dims up
    to 128.  Decode-shaped calls that probjax's FLOP rule (:616-620) finds
    cheaper absorbed run absorbed on the latent decode kernel (no gradient
    needed, bf16, no bias, ``None`` / ``KVLenMask`` / one-row
    ``KeyPaddingMask``, rank 128 / 512 / 576, ``Lq * H <= 128``); the rest
    materialise.  Dropout raises ``ValueError``.
    """
    del rng, unused_tuning
    if q.ndim != 4:
        raise ValueError(f"q must be rank 4 [B,Q,H,D], got shape {tuple(q.shape)}")
    if cache.ndim != 3:
        raise ValueError(f"cache must be rank 3 [B,S,R], got shape {tuple(cache.shape)}")
    if q.shape[0] != cache.shape[0]:
        raise ValueError(f"batch mismatch: q has {q.shape[0]}, cache has {cache.shape[0]}")
    if (wk is None) != (wv is None):
        raise ValueError(
            "provide both wk and wv (materialized) or neither (absorbed); "
            "mixing the two is not supported"
        )
    if wk is None and q.shape[-1] != cache.shape[-1]:
        raise ValueError(
            "absorbed mode (wk=None) requires qk_head_dim == kv_lora_rank "
            f"({q.shape[-1]} != {cache.shape[-1]})"
        )
    if wk is not None and tuple(wk.shape) != (q.shape[-2], q.shape[-1], cache.shape[-1]):
        raise ValueError(f"wk must be {(q.shape[-2], q.shape[-1], cache.shape[-1])}, got {tuple(wk.shape)}")
    if wv is not None and (wv.ndim != 3 or wv.shape[0] != q.shape[-2] or wv.shape[2] != cache.shape[-1]):
        raise ValueError(f"wv must be [heads, v_head_dim, {cache.shape[-1]}], got {tuple(wv.shape)}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    if wk is not None:
        if dropout_rate > 0:
            raise ValueError("the HIP latent-attention kernels take no dropout")
        lengths = _mla_absorbed_lengths(q, cache, wk, wv, mask, bias)
        if lengths is not None:
            return _mla_absorbed(q, cache, wk, wv, lengths, sm_scale)
        return _mla_materialized(q, cache, wk, wv, mask=mask, bias=bias, sm_scale=sm_scale)
    if dropout_rate > 0:
        raise ValueError("the HIP latent-attention kernels take no dropout")
    if not hip_device(q) or cache.device != q.device:
        raise ValueError(f"the HIP latent-attention kernels need tensors on a {HIP_ARCH} ROCm device")
    R = q.shape[-1]
    dv = R if v_dim is None else int(v_dim)
    if not 1 <= dv <= R:
        raise ValueError(f"v_dim must be in [1, {R}], got {dv}")
    lengths = _latent_decode_lengths(q, cache, mask, bias, dv)
    if lengths is not None:
        rk, dvk = _mla_decode_shape(R, dv)
        qk, ck = (q, cache) if rk == R else (_pad_features(q, rk), _pad_features(cache, rk))
        out = hip.mla_decode(qk, ck, sm_scale=float(sm_scale), v_dim=dvk,
                             kv_lengths=None if isinstance(lengths, str) else lengths)
        return out if dvk == dv else out[..., :dv]
    return _mla_latent(q, cache, mask=mask, bias=bias, sm_scale=float(sm_scale), v_dim=dv)


def _latent_decode_lengths(q, cache, mask, bias, dv):
    """Per-batch KV lengths ("all" for none) when an absorbed call is a decode
    step the split-KV latent kernel computes exactly (no gradient, no bias,
    ``None`` / ``KVLenMask`` / one-row ``KeyPaddingMask``, bf16 / fp16, a rank and
    output width it carries (zero-padded up to the next kernel rank,
    ``_mla_decode_shape``), ``Lq * H <= 128``); else None."""
    B, l_q, H, R = q.shape
    if bias is not None or _needs_grad(q, cache):
        return None
    if q.dtype != cache.dtype or q.dtype not in HALF_DTYPES:
        return None
    if _mla_decode_shape(R, dv) is None or l_q * H > MLA_DECODE_MAX_ROWS:
        return None
    lm = lower_mask(mask)
    if lm is None:
        return None
    if lm.row_kv_lengths is not None and l_q == 1:
        rows = _row_kv_lengths(lm.row_kv_lengths, B, 1, q.device)
        if rows is None:
            return None
        lm.row_kv_lengths, lm.kv_lengths = None, rows[:, 0]
    if lm.causal or lm.extended or lm.q_valid is not None or lm.kv_valid is not None:
        return None
    if lm.kv_lengths is None:
        return "all"
    return _lengths_tensor(lm.kv_lengths, B, q.device)


def _latent_width(r: int, dtype):
    """The kernel rank that carries latent width ``r`` (zero-padded): a flash
    head width up to 256, else 512 or 576 (bfloat16 / float16); None when too wide."""
    w = _kernel_width(r, dtype)
    if w is not None:
        return w
    if dtype not in HALF_DTYPES:
        return None
    return next((x for x in LATENT_WIDTHS if x >= r), None)


class _LatentFunction(torch.autograd.Function):
    """Absorbed latent attention on the wide latent kernels, differentiable in
    ``q`` and ``cache``: the forward is ``pjx_mla_fwd``, the backward
    ``pjx_mla_bwd`` (probjax's custom VJP of ``mla``, latent_attention.py:
    752-766: the VJP of ``mha`` over K = V = the latent broadcast to every
    head, so the cache gets the head sum of dK + dV; the bias none)."""

    @staticmethod
    def forward(ctx, q, cache, st):
        o, lse = hip.mla_fwd(q, cache, sm_scale=st["sm_scale"], v_dim=st["dv"], return_lse=True, **st["plan"])
        ctx.save_for_backward(q, cache, o, lse)
        ctx.st = st
        return o

    @staticmethod
    def backward(ctx, dout):
        q, cache, o, lse = ctx.saved_tensors
        st = ctx.st
        dq, dc = hip.mla_bwd(q, cache, o, dout.to(o.dtype), lse, sm_scale=st["sm_scale"], **st["plan"])
        return dq, dc, None


def _mla_latent(q, cache, *, mask, bias, sm_scale, v_dim):
    """Absorbed ``mla`` for any query length, mask and bias (latent_attention.py:
    79-197, 636-766), with the reference's gradient.  Latent widths up to 256
    run the flash kernels with the latent as one shared K = V head (torch
    autograd adds the dK and dV of that one tensor); 512 and 576 (bfloat16 / float16)
    run the wide latent kernels.  A width between kernel ranks is zero-padded
    (zero features change no score and add zero output columns)."""
    B, l_q, H, R = q.shape
    if q.dtype != cache.dtype:
        raise ValueError(f"q and cache must share a dtype, got {q.dtype} and {cache.dtype}")
    width = _latent_width(R, q.dtype)
    if width is None:
        raise ValueError(f"absorbed mla supports latent widths up to {FLASH_HEAD_DIMS_F32[-1]} in float32 and "
                         f"{LATENT_WIDTHS[-1]} in bfloat16 / float16, got {R} ({q.dtype})")
    if width <= FLASH_HEAD_DIMS[-1]:
        c4 = cache[:, :, None, :]
        e = _eligible(q, c4, c4, mask=mask, bias=bias, dropout_rate=0.0)
        out = None if e is None else _run(q, c4, c4, e[0], e[1], sm_scale, False)
        if out is None:
            raise ValueError("the HIP latent-attention kernels cannot compute this call exactly: "
                             + _unsupported_message(q, c4, mask, bias, 0.0))
        return out if v_dim == R else out[..., :v_dim]
    qp = q if width == R else _pad_features(q, width)
    cp = cache if width == R else _pad_features(cache, width)
    cp4 = cp[:, :, None, :]
    e = _eligible(qp, cp4, cp4, mask=mask, bias=bias, dropout_rate=0.0)
    plan = None if e is None else _flash_plan(qp, cp4, cp4, e[0], e[1], check_dim=False)
    if plan is None:
        raise ValueError("the HIP latent-attention kernels cannot compute this call exactly: "
                         + _unsupported_message(qp, cp4, mask, bias, 0.0))
    dvk = 512 if v_dim <= 512 else 576
    st = dict(sm_scale=sm_scale, dv=dvk, plan=plan)
    if not _needs_grad(q, cache):
        with torch.no_grad():
            out = hip.mla_fwd(qp, cp, sm_scale=sm_scale, v_dim=dvk, **plan)
    else:
        out = _LatentFunction.apply(qp, cp, st)
    return out if v_dim == dvk else out[..., :v_dim]


# ---------------------------------------------------------------------------
# Dispatchers (probjax.nn.layers.attention)
# ---------------------------------------------------------------------------

def flex_attention(query, key, value, mask=None, bias=None, dropout_rng=None,
                   dropout_rate: float = 0.0, broadcast_dropout: bool = False,
                   deterministic=True, dtype=None, precision=None, module=None,
                   sm_scale: float | None = None, enable_gqa: bool = False,
                   split_kv: bool | None = None, implementation: str | None = None,
                   _bias_grad: bool = False, _flax_fill: bool = False, **unused_tuning):
    """Fused softmax attention with mask/bias objects (probjax
    ``flex_attention``, layers/attention.py:1426-1759).

    ``implementation``: ``None`` (the device table: the HIP route on gfx950
    unless ``PROBJAX_ATTENTION_HIP=0``) or ``"hip"`` (forced; ``ValueError``
    when the kernels cannot compute the call exactly).  Rank-3 inputs get a
    leading batch axis; ``sm_scale`` defaults to ``1/sqrt(D)``.
    """
    del dropout_rng, broadcast_dropout, precision, module, unused_tuning
    if dtype is not None:
        query, key, value = (x.to(dtype) for x in (query, key, value))
    if (query.dtype != key.dtype) or (query.dtype != value.dtype):
        raise ValueError(
            f"Expected query, key, and value to have the same dtype, "
            f"but got query.dtype: {query.dtype}, key.dtype: {key.dtype}, "
            f"and value.dtype: {value.dtype} instead."
        )
    if (query.ndim < 3) or (key.ndim < 3) or (value.ndim < 3):
        raise ValueError(
            f"Expected query, key, and value to all be at least 3 dimensional, but got query.ndim: "
            f"{query.ndim}, key.ndim: {key.ndim}, and value.ndim: {value.ndim} instead."
        )
    if (not enable_gqa) and query.shape[-2] != key.shape[-2]:
        raise ValueError(
            f"Expect query and key/value to have the same number of heads "
            f"but got Hq={query.shape[-2]} and Hkv={key.shape[-2]}. "
            f"Try setting enable_gqa=True for GQA."
        )
    if enable_gqa and query.shape[-2] % key.shape[-2] != 0:
        raise ValueError(
            f"Expect number of query heads to be a multiple of kv heads for GQA "
            f"but got Hq={query.shape[-2]} and Hkv={key.shape[-2]}."
        )
    if implementation not in (None, "hip"):
        raise ValueError(f"implementation must be None or 'hip', got {implementation!r}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(query.shape[-1])
    squeeze = query.ndim == 3
    if squeeze:
        query, key, value = query[None], key[None], value[None]
    active_dropout = dropout_rate if not deterministic and dropout_rate > 0 else 0.0
    out = None
    low_rank, rest = split_low_rank_bias(bias)
    out_dim = None
    if low_rank:
        folded = _fold_low_rank(query, key, value, low_rank, float(sm_scale))
        if folded is None:
            raise ValueError(
                f"implementation={implementation!r}: head_dim {query.shape[-1]} plus the low-rank "
                f"bias ranks {[t.rank for t in low_rank]} exceeds the kernels' {FLASH_HEAD_DIMS[-1]}")
        query, key, value, out_dim = folded
        bias = rest
    e = _eligible(query, key, value, mask=mask, bias=bias, dropout_rate=active_dropout)
    if e is not None and (implementation == "hip" or device_table_enabled()):
        out = _run(query, key, value, e[0], e[1], float(sm_scale), split_kv, bias_grad=_bias_grad,
                   want_lse=_flax_fill)
        if out is not None and _flax_fill:
            out = _flax_empty_rows(out[0], out[1], value)
    if out is None:
        raise ValueError(
            f"implementation={implementation!r}: "
            + _unsupported_message(query, key, mask, bias, active_dropout)
            + ("" if implementation == "hip" or device_table_enabled()
               else " (the HIP route is switched off by PROBJAX_ATTENTION_HIP=0)")
        )
    if out_dim is not None:
        out = out[..., :out_dim]
    return out[0] if squeeze else out


def _flax_empty_rows(out, lse, value):
    """Flax's output for rows whose keys are all masked: ``where(mask,
    logits, big_neg)`` gives such a row equal weights over every key, so the
    mean of V (and dV = dO / Lk through autograd; no gradient reaches q, k or
    the bias there).  The kernels leave such rows at zero with ``lse = +inf``,
    so the fill is one device-side select, with no host synchronisation.
    With no keys at all the einsum over an empty key axis gives zeros, which
    the kernels already return."""
    l_k = value.shape[1]
    if l_k == 0:
        return out
    empty = torch.isinf(lse).transpose(1, 2)[..., None]  # [B, Lq, Hq, 1]
    vmean = value.float().mean(dim=1)  # [B, Hkv, Dv]
    vmean = vmean.repeat_interleave(out.shape[2] // vmean.shape[1], dim=1)[:, None]
    if vmean.shape[-1] != out.shape[-1]:
        vmean = vmean[..., : out.shape[-1]]
    return torch.where(empty, vmean.to(out.dtype), out)


def _fold_low_rank(query, key, value, terms, sm_scale: float):
    """Low-rank bias terms folded into Q/K (probjax ``flex_attention``,
    layers/attention.py:1600-1635): each term's factors, scaled by
    ``sqrt(scale / sm_scale)`` in the input dtype, are appended to the query
    and key features (V gets zero features), so ``sm_scale * q'.k'`` carries
    ``scale * U.V``; K/V are repeated to the query heads first.  The features
    are zero-padded to a kernel head dim.  Returns ``(q', k', v', output
    width)``, or None when the folded head dim exceeds the kernels'.  Torch
    autograd carries the gradients of the concatenation to the factors."""
    if sm_scale <= 0:
        raise ValueError("LowRankBias requires a positive sm_scale")
    hq = query.shape[-2]
    if key.shape[-2] != hq:
        rep = hq // key.shape[-2]
        key = key.repeat_interleave(rep, dim=-2)
        value = value.repeat_interleave(rep, dim=-2)
    q_extra, k_extra = [], []
    for t in terms:
        qf, kf = t.factors(query.shape[-3], key.shape[-3], hq, dtype=query.dtype)
        f = math.sqrt(t.scale / sm_scale)
        q_extra.append(qf.to(query.device).expand(tuple(query.shape[:-1]) + (t.rank,)) * f)
        k_extra.append(kf.to(key.device).expand(tuple(key.shape[:-1]) + (t.rank,)) * f)
    extra = sum(x.shape[-1] for x in q_extra)
    width = _kernel_width(query.shape[-1] + extra, query.dtype)
    if width is None:
        return None
    pad = width - query.shape[-1] - extra

    def zeros(like, n):
        return like.new_zeros(tuple(like.shape[:-1]) + (n,))

    out_dim = value.shape[-1]
    query = torch.cat((query, *q_extra, zeros(query, pad)), dim=-1)
    key = torch.cat((key, *k_extra, zeros(key, pad)), dim=-1)
    value = torch.cat((value, zeros(value, width - out_dim)), dim=-1)
    return query, key, value, out_dim


# probjax's fused route of dot_product_attention (layers/attention.py:1161-1164):
# position-only masks and at least this many keys; other calls take Flax's einsum.
_FUSED_MASKS = ("NoMask", "CausalMask", "LocalWindowMask", "CausalLocalWindowMask")
_FUSED_MIN_KV_LEN = 64


def dot_product_attention(query, key, value, mask=None, bias=None, dropout_rng=None,
                          dropout_rate: float = 0.0, broadcast_dropout: bool = False,
                          deterministic=True, dtype=None, precision=None, module=None,
                          sm_scale: float | None = None, enable_gqa: bool = False,
                          implementation: str | None = None):
    """Softmax attention with Flax ``dot_product_attention`` semantics (probjax
    layers/attention.py:1205-1319) on the HIP kernels: leading batch dims are
    flattened, K/V may have fewer heads (GQA), ``sm_scale`` defaults to
    ``1/sqrt(D)``.  ``implementation`` in ``(None, "hip")``.  A ``DenseBias``
    whose tensor requires grad receives its gradient, as in probjax's dense
    path (``flex_attention`` / ``mha`` give bias data no cotangent, as the
    reference's kernel VJP does).  Flax-style arrays are taken too: a boolean
    ``mask`` (True = attend) and an additive ``bias``, broadcastable to
    ``batch + [H, Lq, Lk]`` (probjax hands them to Flax's einsum,
    layers/attention.py:1298-1319).

    Rows whose keys the mask drops entirely follow the reference's two
    paths.  probjax takes its fused kernel only for no mask or a
    position-only mask (``NoMask``, ``CausalMask``, ``LocalWindowMask``,
    ``CausalLocalWindowMask``), no bias, no ``module`` / ``precision`` and at
    least 64 keys (``_use_fused_gpu_attention``, layers/attention.py:1161-1202;
    the device routes refuse a bias, attention_device.py:128); every other
    call runs Flax's einsum over ``mask.dense()``, whose masking by the
    dtype's most negative value gives such a row equal weights over every key:
    the mean of V.  On the fused route the kernel's zeros stand, as in
    ``flex_attention``.
    """
    if implementation not in (None, "hip"):
        raise ValueError(f"implementation must be None or 'hip', got {implementation!r}")
    batch_shape = tuple(query.shape[:-3])
    flat = [x.reshape((-1,) + tuple(x.shape[-3:])) for x in (query, key, value)]
    flax_path = (bias is not None or isinstance(mask, torch.Tensor) or module is not None
                 or precision is not None or key.shape[-3] < _FUSED_MIN_KV_LEN
                 or (mask is not None and type(mask).__name__ not in _FUSED_MASKS))
    if isinstance(mask, torch.Tensor) or isinstance(bias, torch.Tensor):
        mask, bias = _flax_arrays(mask, bias, batch_shape, flat[0], flat[1])
    out = flex_attention(*flat, mask=mask, bias=bias, dropout_rng=dropout_rng,
                         dropout_rate=dropout_rate, deterministic=deterministic, dtype=dtype,
                         sm_scale=sm_scale, enable_gqa=enable_gqa or query.shape[-2] != key.shape[-2],
                         implementation=implementation, _bias_grad=True, _flax_fill=flax_path)
    return out.reshape(batch_shape + tuple(out.shape[-3:]))


def _flax_arrays(mask, bias, batch_shape, q, k):
    """Flax array mask / bias (layers/attention.py:1298-1319 hands arrays to
    ``flax.linen.dot_product_attention``): a boolean ``mask`` (True = attend)
    and an additive ``bias``, each broadcastable to ``batch + [H, Lq, Lk]``.
    Returns ``(mask object, bias object)``: the bias as a ``DenseBias``
    ``[B, H|1, Lq, Lk]`` over the flattened batch (its tensor keeps its
    autograd history) and the mask as a 0 / -inf ``DenseBias`` term.  Rows
    the mask drops entirely are found from the kernels' ``+inf`` LSE."""
    from .masks import AttentionBias, DenseBias

    B, l_q, h_q = q.shape[0], q.shape[1], q.shape[2]
    l_k = k.shape[1]

    def dense(x, what):
        t = torch.as_tensor(x, device=q.device)
        if t.ndim < 2:
            raise ValueError(f"array {what} needs at least [Lq, Lk] dims, got shape {tuple(t.shape)}")
        t = t.reshape((1,) * max(0, len(batch_shape) + 3 - t.ndim) + tuple(t.shape))
        heads = t.shape[-3]
        if heads not in (1, h_q):
            raise ValueError(f"array {what} has {heads} heads for {h_q} query heads")
        try:
            t = t.expand(batch_shape + (heads, l_q, l_k))
        except RuntimeError as e:
            raise ValueError(f"array {what} of shape {tuple(x.shape)} does not broadcast to "
                             f"{batch_shape + (h_q, l_q, l_k)}") from e
        return t.reshape((B, heads, l_q, l_k))

    terms = []
    if isinstance(bias, torch.Tensor):
        terms.append(dense(bias, "bias").float())
        bias = None
    if isinstance(mask, torch.Tensor):
        keep = dense(mask, "mask").bool()
        terms.append(torch.zeros(keep.shape, device=q.device).masked_fill_(~keep, float("-inf")))
        mask = None
    if terms:
        extra = DenseBias(terms[0] if len(terms) == 1 else terms[0] + terms[1])
        bias = extra if bias is None else (bias + extra if isinstance(bias, AttentionBias) else extra)
    return mask, bias
