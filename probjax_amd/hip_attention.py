"""Device-tensor wrappers over the C ABI (torch provides HBM buffers and streams).

Each function validates shapes/dtypes on the host (``ValueError`` for what the
kernels do not take), allocates the outputs, and enqueues the kernels on the
tensors' current HIP stream.  Inputs must already be resident on one ROCm
device; nothing is copied between host and device.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import torch

from . import native

_DTYPES = {
    torch.bfloat16: native.PJX_DTYPE_BF16,
    torch.float16: native.PJX_DTYPE_F16,
    torch.float32: native.PJX_DTYPE_F32,
}
# the dtypes of the 16-bit (MFMA bf16 / fp16) kernels
HALF_DTYPES = (torch.bfloat16, torch.float16)


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; expected bfloat16, float16 or float32") from None


def _half_code(who: str, *ts) -> int:
    """Dtype code of tensors that must share one 16-bit dtype."""
    if ts[0].dtype not in HALF_DTYPES or any(t.dtype != ts[0].dtype for t in ts):
        raise ValueError(f"{who} takes bfloat16 or float16 tensors of one dtype")
    return _DTYPES[ts[0].dtype]


def _on_device(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            raise ValueError("the HIP attention kernels need tensors on a ROCm device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _lengths(kv_lengths, batch, dev):
    if kv_lengths is None:
        return None
    L = torch.as_tensor(kv_lengths, device=dev).reshape(-1).to(torch.int32).contiguous()
    if L.numel() != batch:
        raise ValueError(f"kv_lengths has {L.numel()} entries for batch {batch}")
    return L


@dataclass
class ScoreModsArgs:
    """Extended masks and score modifiers of the flash kernels
    (``pjx_score_mods``): device tensors, or None / defaults for absent."""

    causal_shift: int = 0  # with causal: k <= q + causal_shift
    window_left: int = -1  # >= 0: k >= q - window_left
    window_right: int = -1  # >= 0: k <= q + window_right
    prefix_lengths: torch.Tensor | None = None  # [B] int32
    seq_lengths: torch.Tensor | None = None  # [B] int32
    segment_q: torch.Tensor | None = None  # [B, Lq] int32
    segment_k: torch.Tensor | None = None  # [B, Lk] int32
    alibi_slopes: torch.Tensor | None = None  # [Hq] float32
    alibi_symmetric: bool = False
    softcap: float = 0.0
    head_scales: torch.Tensor | None = None  # [Hq] float32
    constant: float = 0.0
    row_kv_lengths: torch.Tensor | None = None  # [B, Lq] int32: k < row_kv_lengths[b, q]


def _mods_struct(m: ScoreModsArgs | None, B, Lq, Lk, Hq, dev):
    """``pjx_score_mods`` for the call (shapes and dtypes checked), or None."""
    if m is None:
        return None

    def dev_tensor(t, shape, dtype, what):
        if t is None:
            return None
        if not isinstance(t, torch.Tensor) or t.device != dev or t.dtype != dtype:
            raise ValueError(f"{what} must be a {dtype} tensor on {dev}")
        if tuple(t.shape) != shape:
            raise ValueError(f"{what} must have shape {shape}, got {tuple(t.shape)}")
        return t.contiguous()

    ts = {
        "prefix_lengths": dev_tensor(m.prefix_lengths, (B,), torch.int32, "prefix_lengths"),
        "seq_lengths": dev_tensor(m.seq_lengths, (B,), torch.int32, "seq_lengths"),
        "segment_q": dev_tensor(m.segment_q, (B, Lq), torch.int32, "segment_q"),
        "segment_k": dev_tensor(m.segment_k, (B, Lk), torch.int32, "segment_k"),
        "alibi_slopes": dev_tensor(m.alibi_slopes, (Hq,), torch.float32, "alibi_slopes"),
        "head_scales": dev_tensor(m.head_scales, (Hq,), torch.float32, "head_scales"),
        "row_kv_lengths": dev_tensor(m.row_kv_lengths, (B, Lq), torch.int32, "row_kv_lengths"),
    }
    st = native.ScoreMods(
        causal_shift=int(m.causal_shift), window_left=int(m.window_left),
        window_right=int(m.window_right), alibi_symmetric=int(bool(m.alibi_symmetric)),
        softcap=float(m.softcap), constant=float(m.constant),
        **{k: (None if v is None else v.data_ptr()) for k, v in ts.items()},
    )
    return st, ts  # the tensors stay alive for the call


def flash_attention_fwd(
    q, k, v, *, sm_scale: float, causal: bool = False, kv_lengths=None, bias=None,
    q_valid: int | None = None, kv_valid: int | None = None, return_lse: bool = False,
    mods: ScoreModsArgs | None = None,
):
    """``pjx_flash_fwd``: ``q [B, Lq, Hq, D]``, ``k/v [B, Lk, Hkv, D]`` -> ``o``.

    ``bias`` is fp32 ``[1|B, 1|Hq, Lq, Lk]``; ``kv_lengths`` int ``[B]``;
    ``q_valid``/``kv_valid`` are static query/key lengths (QKVLengthMask).
    Returns ``o`` (and the natural-log LSE ``[B, Hq, Lq]`` with ``return_lse``).
    ``mods``: extended masks / score modifiers.
    """
    dev = _on_device(q, k, v, bias)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be [B, T, H, D]")
    B, Lq, Hq, D = q.shape
    _, Lk, Hkv, Dk = k.shape
    if k.shape != v.shape or k.shape[0] != B or Dk != D:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share a dtype")
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} must be a multiple of kv heads {Hkv}")
    if D not in (64, 128, 256):
        raise ValueError(f"head_dim {D} not supported (64, 128 or 256)")
    if not sm_scale > 0:
        raise ValueError("sm_scale must be > 0")
    code = _dtype_code(q)
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    bb = bh = 1
    if bias is not None:
        if bias.ndim != 4 or tuple(bias.shape[-2:]) != (Lq, Lk):
            raise ValueError(f"bias must be [1|B, 1|H, {Lq}, {Lk}], got {tuple(bias.shape)}")
        bb, bh = bias.shape[:2]
        if bb not in (1, B) or bh not in (1, Hq):
            raise ValueError(f"bias {tuple(bias.shape)} does not broadcast to B={B}, H={Hq}")
        bias = bias.to(torch.float32).contiguous()
    L = _lengths(kv_lengths, B, dev)
    ms = _mods_struct(mods, B, Lq, Lk, Hq, dev)
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq, Lq), dtype=torch.float32, device=dev) if return_lse else None
    lib = native.load()
    rc = lib.pjx_flash_fwd(
        code, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(L), _ptr(bias), bb, bh,
        B, Lq, Lk, Hq, Hkv, D, Lq if q_valid is None else int(q_valid),
        Lk if kv_valid is None else int(kv_valid), int(bool(causal)), float(sm_scale),
        None if ms is None else ctypes.byref(ms[0]), _stream(dev),
    )
    native.check(rc)
    return (o, lse) if return_lse else o


def flash_attention_bwd(
    q, k, v, o, do, lse, *, sm_scale: float, causal: bool = False, kv_lengths=None, bias=None,
    q_valid: int | None = None, kv_valid: int | None = None, workspace=None,
    mods: ScoreModsArgs | None = None, bias_grad: bool = False, ds_route: bool | None = None,
):
    """``pjx_flash_bwd``: gradients ``(dq, dk, dv)`` of ``flash_attention_fwd``
    (and, with ``bias_grad``, ``dbias``: dL/d(bias) summed to the bias's own
    ``[1|B, 1|H, Lq, Lk]`` shape, fp32).

    ``o`` and ``lse`` are the forward's output and natural-log LSE; ``do`` the
    output gradient.  Masks, bias and scale must be the forward's.  bf16, fp16 or fp32.

    ``ds_route`` (when ``workspace`` is None): the workspace this call
    allocates.  None sizes it for the dS route (dQ from the rounded dS the
    dK/dV kernel keeps, ``pjx_flash_bwd_ds_workspace_size``) where the route
    exists (16-bit, head dim 256 -- after padding -- without bias or score
    modifiers) and its ``2 * B * Hq * Lq' * Lk'`` bytes of dS fit the budget
    (``_ds_budget``); True takes it whatever its size (ValueError where it
    does not exist); False never does.
    """
    dev = _on_device(q, k, v, o, do, lse, bias)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, v must be [B, T, H, D]")
    B, Lq, Hq, D = q.shape
    _, Lk, Hkv, Dk = k.shape
    if k.shape != v.shape or k.shape[0] != B or Dk != D:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, k {tuple(k.shape)}, v {tuple(v.shape)}")
    if o.shape != q.shape or do.shape != q.shape or tuple(lse.shape) != (B, Hq, Lq):
        raise ValueError("o and do must be shaped like q and lse [B, Hq, Lq]")
    if not (q.dtype == k.dtype == v.dtype == o.dtype == do.dtype):
        raise ValueError("q, k, v, o, do must share a dtype")
    code = _dtype_code(q)
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} must be a multiple of kv heads {Hkv}")
    if D not in (64, 128, 256):
        raise ValueError(f"head_dim {D} not supported (64, 128 or 256)")
    if not sm_scale > 0:
        raise ValueError("sm_scale must be > 0")
    q, k, v, o, do = (t.contiguous() for t in (q, k, v, o, do))
    lse = lse.to(torch.float32).contiguous()
    bb = bh = 1
    if bias is not None:
        if bias.ndim != 4 or tuple(bias.shape[-2:]) != (Lq, Lk):
            raise ValueError(f"bias must be [1|B, 1|H, {Lq}, {Lk}], got {tuple(bias.shape)}")
        bb, bh = bias.shape[:2]
        if bb not in (1, B) or bh not in (1, Hq):
            raise ValueError(f"bias {tuple(bias.shape)} does not broadcast to B={B}, H={Hq}")
        bias = bias.to(torch.float32).contiguous()
    L = _lengths(kv_lengths, B, dev)
    ms = _mods_struct(mods, B, Lq, Lk, Hq, dev)
    if bias_grad and bias is None:
        raise ValueError("bias_grad needs the bias")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dbias = torch.zeros((B, Hq, Lq, Lk), dtype=torch.float32, device=dev) if bias_grad else None
    lib = native.load()
    nbytes = int(lib.pjx_flash_bwd_workspace_size(B, Hq, Lq))
    if workspace is None:
        ds_bytes = 0
        if bias is None and ms is None:
            ds_bytes = int(lib.pjx_flash_bwd_ds_workspace_size(code, B, Hq, Lq, Lk, D))
        nbytes = _ds_route_bytes(nbytes, ds_bytes, ds_route, dev,
                                 "the dS route takes 16-bit inputs at head dim 256 without bias or score modifiers")
    ws = _workspace(nbytes, dev, workspace)
    rc = lib.pjx_flash_bwd(
        code, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(do), _ptr(lse), _ptr(dq),
        _ptr(dk), _ptr(dv), _ptr(dbias), _ptr(ws), ws.numel(), _ptr(L), _ptr(bias), bb, bh, B, Lq, Lk, Hq, Hkv, D,
        Lq if q_valid is None else int(q_valid), Lk if kv_valid is None else int(kv_valid),
        int(bool(causal)), float(sm_scale), None if ms is None else ctypes.byref(ms[0]), _stream(dev),
    )
    native.check(rc)
    if dbias is None:
        return dq, dk, dv
    dims = [d for d, n in ((0, bb), (1, bh)) if n == 1]
    if dims:
        dbias = dbias.sum(dim=dims, keepdim=True)
    return dq, dk, dv, dbias


def _ds_budget(dev) -> int:
    """Bytes of dS a backward call may keep in its workspace (the dS route):
    ``PJX_BWD_DS_MAX_BYTES`` if set, else 1/16 of the device's memory, at most
    16 GiB."""
    env = os.environ.get("PJX_BWD_DS_MAX_BYTES")
    if env:
        return int(env)
    total = torch.cuda.get_device_properties(dev).total_memory
    return min(total // 16, 16 << 30)


def _ds_route_bytes(base: int, ds_bytes: int, ds_route, dev, why: str) -> int:
    """Workspace bytes a backward call allocates: ``ds_bytes`` (the dS route,
    0 where it does not exist) when ``ds_route`` is True, or None and the dS
    part fits ``_ds_budget``; else ``base``."""
    if ds_route and not ds_bytes:
        raise ValueError(why)
    if ds_bytes and ds_route is not False and (ds_route or ds_bytes - base <= _ds_budget(dev)):
        return ds_bytes
    return base


def decode_workspace_bytes(batch, groups, rows, kv_len, v_dim, chunk=0) -> int:
    return int(native.load().pjx_decode_workspace_size(batch, groups, rows, kv_len, v_dim, chunk))


def _workspace(nbytes, dev, workspace):
    if workspace is None:
        return torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=dev)
    if workspace.device != dev or workspace.numel() * workspace.element_size() < nbytes:
        raise ValueError(f"workspace must hold {nbytes} bytes on {dev}")
    return workspace


def splitkv_decode(
    q, k, v, *, sm_scale: float, kv_lengths=None, chunk: int = 0, return_lse: bool = False,
    workspace=None,
):
    """``pjx_splitkv_decode``: bf16, fp16 or fp32 ``q [B, Lq, Hq, D]``,
    ``k [B, S, Hkv, D]``, ``v [B, S, Hkv, Dv]`` -> ``o [B, Lq, Hq, Dv]``; D and
    Dv each 64, 128 or 256, any number of packed rows ``(Hq/Hkv)*Lq``."""
    dev = _on_device(q, k, v)
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4 or k.shape[:3] != v.shape[:3]:
        raise ValueError("q must be [B, Lq, Hq, D], k [B, S, Hkv, D] and v [B, S, Hkv, Dv]")
    B, Lq, Hq, D = q.shape
    _, S, Hkv, Dk = k.shape
    Dv = v.shape[-1]
    if Dk != D or k.shape[0] != B or Hq % Hkv:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, k {tuple(k.shape)}")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("split-KV decode takes bfloat16, float16 or float32 q, k, v of one dtype")
    if D not in (64, 128, 256) or Dv not in (64, 128, 256):
        raise ValueError(f"split-KV decode needs head dims 64, 128 or 256, got D={D}, Dv={Dv}")
    rows = (Hq // Hkv) * Lq
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    L = _lengths(kv_lengths, B, dev)
    nbytes = decode_workspace_bytes(B, Hkv, rows, S, Dv, chunk)
    ws = _workspace(nbytes, dev, workspace)
    o = torch.empty((B, Lq, Hq, Dv), dtype=q.dtype, device=dev)
    lse = torch.empty((B, Hq, Lq), dtype=torch.float32, device=dev) if return_lse else None
    rc = native.load().pjx_splitkv_decode(
        _dtype_code(q), _ptr(q), _ptr(k), _ptr(v), _ptr(L), _ptr(o), _ptr(lse), _ptr(ws),
        nbytes, B, Lq, S, Hq, Hkv, D, Dv, float(sm_scale), int(chunk), _stream(dev),
    )
    native.check(rc)
    return (o, lse) if return_lse else o


# (rank, v_dim) pairs of the latent decode kernel (any number of folded rows).
MLA_DECODE_SHAPES = ((576, 512), (576, 576), (512, 512), (256, 256), (128, 128), (64, 64))


def mla_decode(
    q, cache, *, sm_scale: float, v_dim: int | None = None, kv_lengths=None, chunk: int = 0,
    return_lse: bool = False, workspace=None,
):
    """``pjx_mla_decode``: bf16 / fp16 ``q [B, Lq, H, R]`` over ``cache [B, S, R]`` (K = V)."""
    dev = _on_device(q, cache)
    if q.ndim != 4 or cache.ndim != 3:
        raise ValueError("q must be [B, Lq, H, R] and cache [B, S, R]")
    B, Lq, H, R = q.shape
    if cache.shape[0] != B or cache.shape[2] != R:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, cache {tuple(cache.shape)}")
    code = _half_code("MLA decode", q, cache)
    dv = R if v_dim is None else int(v_dim)
    if (R, dv) not in MLA_DECODE_SHAPES:
        raise ValueError(f"MLA decode supports (R, v_dim) in {MLA_DECODE_SHAPES}; got ({R}, {dv})")
    S = cache.shape[1]
    q, cache = q.contiguous(), cache.contiguous()
    L = _lengths(kv_lengths, B, dev)
    nbytes = decode_workspace_bytes(B, 1, Lq * H, S, dv, chunk)
    ws = _workspace(nbytes, dev, workspace)
    o = torch.empty((B, Lq, H, dv), dtype=q.dtype, device=dev)
    lse = torch.empty((B, H, Lq), dtype=torch.float32, device=dev) if return_lse else None
    rc = native.load().pjx_mla_decode(
        code, _ptr(q), _ptr(cache), _ptr(L), _ptr(o), _ptr(lse), _ptr(ws),
        nbytes, B, Lq, H, S, R, dv, float(sm_scale), int(chunk), _stream(dev),
    )
    native.check(rc)
    return (o, lse) if return_lse else o


def mla_fwd(
    q, cache, *, sm_scale: float, v_dim: int | None = None, causal: bool = False, kv_lengths=None,
    bias=None, q_valid: int | None = None, kv_valid: int | None = None, return_lse: bool = False,
    mods: ScoreModsArgs | None = None,
):
    """``pjx_mla_fwd``: absorbed latent attention ``q [B, Lq, H, R]`` over
    ``cache [B, S, R]`` (K = V = cache) -> ``o [B, Lq, H, v_dim]`` (the first
    ``v_dim`` columns; ``None`` = R), any query length, with the masks, bias
    and modifiers of ``flash_attention_fwd`` (bias ``[1|B, 1|H, Lq, S]``)."""
    dev = _on_device(q, cache, bias)
    if q.ndim != 4 or cache.ndim != 3:
        raise ValueError("q must be [B, Lq, H, R] and cache [B, S, R]")
    B, Lq, H, R = q.shape
    if cache.shape[0] != B or cache.shape[2] != R:
        raise ValueError(f"incompatible shapes q {tuple(q.shape)}, cache {tuple(cache.shape)}")
    code = _half_code("the latent flash kernel", q, cache)
    dv = R if v_dim is None else int(v_dim)
    S = cache.shape[1]
    if not sm_scale > 0:
        raise ValueError("sm_scale must be > 0")
    q, cache = q.contiguous(), cache.contiguous()
    bb = bh = 1
    if bias is not None:
        if bias.ndim != 4 or tuple(bias.shape[-2:]) != (Lq, S):
            raise ValueError(f"bias must be [1|B, 1|H, {Lq}, {S}], got {tuple(bias.shape)}")
        bb, bh = bias.shape[:2]
        if bb not in (1, B) or bh not in (1, H):
            raise ValueError(f"bias {tuple(bias.shape)} does not broadcast to B={B}, H={H}")
        bias = bias.to(torch.float32).contiguous()
    L = _lengths(kv_lengths, B, dev)
    ms = _mods_struct(mods, B, Lq, S, H, dev)
    o = torch.empty((B, Lq, H, dv), dtype=q.dtype, device=dev)
    lse = torch.empty((B, H, Lq), dtype=torch.float32, device=dev) if return_lse else None
    rc = native.load().pjx_mla_fwd(
        code, _ptr(q), _ptr(cache), _ptr(o), _ptr(lse), _ptr(L), _ptr(bias), bb, bh,
        B, Lq, S, H, R, dv, Lq if q_valid is None else int(q_valid), S if kv_valid is None else int(kv_valid),
        int(bool(causal)), float(sm_scale), None if ms is None else ctypes.byref(ms[0]), _stream(dev),
    )
    native.check(rc)
    return (o, lse) if return_lse else o


def mla_bwd(
    q, cache, o, do, lse, *, sm_scale: float, causal: bool = False, kv_lengths=None, bias=None,
    q_valid: int | None = None, kv_valid: int | None = None, mods: ScoreModsArgs | None = None,
    workspace=None,
):
    """``pjx_mla_bwd``: ``(dq, dcache)`` of ``mla_fwd`` (absorbed latent, bf16
    or fp16, rank 512 / 576).  ``o`` / ``do`` are the forward output and its gradient
    ``[B, Lq, H, v_dim]``, ``lse`` the forward's natural-log LSE ``[B, H, Lq]``;
    masks, bias and scale must be the forward's."""
    dev = _on_device(q, cache, o, do, lse, bias)
    if q.ndim != 4 or cache.ndim != 3:
        raise ValueError("q must be [B, Lq, H, R] and cache [B, S, R]")
    B, Lq, H, R = q.shape
    S = cache.shape[1]
    dv = o.shape[-1]
    if cache.shape[0] != B or cache.shape[2] != R or tuple(o.shape) != (B, Lq, H, dv) or do.shape != o.shape:
        raise ValueError("incompatible shapes for the latent backward")
    if tuple(lse.shape) != (B, H, Lq):
        raise ValueError(f"lse must be [B, H, Lq] = {(B, H, Lq)}")
    code = _half_code("the latent backward", q, cache, o, do)
    q, cache, o, do = (t.contiguous() for t in (q, cache, o, do))
    lse = lse.to(torch.float32).contiguous()
    bb = bh = 1
    if bias is not None:
        if bias.ndim != 4 or tuple(bias.shape[-2:]) != (Lq, S):
            raise ValueError(f"bias must be [1|B, 1|H, {Lq}, {S}], got {tuple(bias.shape)}")
        bb, bh = bias.shape[:2]
        bias = bias.to(torch.float32).contiguous()
    L = _lengths(kv_lengths, B, dev)
    ms = _mods_struct(mods, B, Lq, S, H, dev)
    lib = native.load()
    ws = _workspace(int(lib.pjx_mla_bwd_workspace_size(B, H, Lq, S, R)), dev, workspace)
    dq = torch.empty_like(q)
    dc = torch.empty_like(cache)
    rc = lib.pjx_mla_bwd(
        code, _ptr(q), _ptr(cache), _ptr(o), _ptr(do), _ptr(lse), _ptr(dq), _ptr(dc),
        _ptr(ws), ws.numel(), _ptr(L), _ptr(bias), bb, bh, B, Lq, S, H, R, dv,
        Lq if q_valid is None else int(q_valid), S if kv_valid is None else int(kv_valid),
        int(bool(causal)), float(sm_scale), None if ms is None else ctypes.byref(ms[0]), _stream(dev),
    )
    native.check(rc)
    return dq, dc


def mla_project(cache, wk, wv, *, width: int):
    """``pjx_mla_project``: ``K = C W_K^T``, ``V = C W_V^T`` per head, zero-padded
    to ``width`` channels -> ``(k, v)`` each ``[B, S, H, width]``
    (latent_attention.py:396-410, 413-468)."""
    dev = _on_device(cache, wk, wv)
    if cache.ndim != 3 or wk.ndim != 3 or wv.ndim != 3:
        raise ValueError("cache must be [B, S, R], wk [H, qk_dim, R] and wv [H, v_dim, R]")
    B, S, R = cache.shape
    H, dk, Rk = wk.shape
    if Rk != R or wv.shape[0] != H or wv.shape[2] != R:
        raise ValueError(f"incompatible shapes cache {tuple(cache.shape)}, wk {tuple(wk.shape)}, wv {tuple(wv.shape)}")
    dv = wv.shape[1]
    if not (cache.dtype == wk.dtype == wv.dtype) or cache.dtype not in _DTYPES:
        raise ValueError("cache, wk and wv must share one dtype (bfloat16, float16 or float32)")
    cache, wk, wv = cache.contiguous(), wk.contiguous(), wv.contiguous()
    k = torch.empty((B, S, H, width), dtype=cache.dtype, device=dev)
    v = torch.empty((B, S, H, width), dtype=cache.dtype, device=dev)
    rc = native.load().pjx_mla_project(
        _DTYPES[cache.dtype], _ptr(cache), _ptr(wk), _ptr(wv), _ptr(k), _ptr(v),
        B, S, H, R, dk, dv, int(width), _stream(dev),
    )
    native.check(rc)
    return k, v
