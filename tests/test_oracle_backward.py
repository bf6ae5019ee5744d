"""Pinning of the backward oracle (numpy restatement of probjax's attention backward).

Each check is independent of the restatement's formulas:
* torch autograd in float64 through an explicit masked softmax (rows without a
  valid key output 0, as in the XLA path) and through torch's
  ``scaled_dot_product_attention`` (``is_causal``, ``enable_gqa``);
* central finite differences in float64 on tiny inputs;
* closed forms: ``sum_k dv = sum_q do`` over rows with a valid key (softmax rows
  sum to one), ``dq = 0`` when every key is the same vector (softmax gradient
  rows sum to zero), exact zeros for masked keys and empty rows;
* bf16 mode within the reference's gradient tolerance of fp32
  (probjax tests/test_attention.py:597-626: atol 2e-2, rtol 1e-2);
* a planted mistake (``delta`` left out) fails the finite differences.
"""

import math

import numpy as np
import pytest
import torch

import oracle
from oracle.backward import attention_backward, preprocess_delta
from tests._helpers import rng_normal


def _torch_grads(q, k, v, do, *, scale, keep=None, bias=None):
    """float64 autograd of softmax attention; rows with no valid key output 0."""
    t = lambda x: torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True)  # noqa: E731
    tq, tk, tv = t(q), t(k), t(v)
    G = q.shape[2] // k.shape[2]
    kr = tk.repeat_interleave(G, dim=2)
    vr = tv.repeat_interleave(G, dim=2)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, kr) * scale
    tb = None
    if bias is not None:
        tb = t(bias)
        s = s + tb
    if keep is not None:
        kt = torch.from_numpy(np.asarray(keep))[:, None]  # [B, 1, Q, K]
        s = s.masked_fill(~kt, -math.inf)
        row_ok = kt.any(-1, keepdim=True)
        s = torch.where(row_ok, s, torch.zeros_like(s))
        p = torch.softmax(s, dim=-1) * row_ok
    else:
        p = torch.softmax(s, dim=-1)
    o = torch.einsum("bhqk,bkhd->bqhd", p, vr)
    o.backward(torch.from_numpy(np.asarray(do, np.float64)))
    _torch_grads.dbias = None if tb is None else tb.grad.numpy()
    return o.detach().numpy(), tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


def _forward(q, k, v, *, mask=None, bias=None, scale, dtype="f32", cdt=np.float64):
    return oracle.xla_attention(q, k, v, mask=mask, bias=bias, sm_scale=scale, strategy="dense",
                                dtype=dtype, compute_dtype=cdt, return_lse=True)


CASES = [
    # B, Lq, Lk, Hq, Hkv, D, causal, lengths, bias
    (2, 9, 9, 4, 2, 6, True, None, False),
    (2, 7, 11, 2, 1, 5, False, [11, 4], True),
    (1, 12, 12, 3, 3, 8, True, [5], True),
    (3, 6, 10, 4, 1, 4, False, [0, 3, 10], False),  # batch 0: every row empty
]


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,D,causal,lengths,has_bias", CASES)
def test_backward_matches_torch_autograd_float64(B, Lq, Lk, Hq, Hkv, D, causal, lengths, has_bias):
    q, k, v, do, bias = rng_normal(1, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D),
                                   (B, Lq, Hq, D), (1, Hq, Lq, Lk))
    scale = 1.0 / math.sqrt(D)
    masks = []
    if causal:
        masks.append(oracle.CausalMask())
    if lengths is not None:
        masks.append(oracle.KVLenMask(np.array(lengths, np.int32)))
    mask = None
    for m in masks:
        mask = m if mask is None else mask & m
    db = oracle.DenseBias(bias) if has_bias else None
    keep = None
    if mask is not None:
        keep = np.stack([np.asarray(mask.tile_keep(b, np.arange(Lq), np.arange(Lk)), bool)
                         for b in range(B)])
    o, lse = _forward(q, k, v, mask=mask, bias=db, scale=scale)
    got = attention_backward(q, k, v, o, do, lse, mask=mask, bias=db, sm_scale=scale,
                             compute_dtype=np.float64, return_dbias=has_bias)
    o_t, *want = _torch_grads(q, k, v, do, scale=scale, keep=keep,
                              bias=bias if has_bias else None)
    if has_bias:
        # dL/d(bias): per query head, summed over the batch the bias [1, H] broadcasts
        want.append(_torch_grads.dbias)
        got = (*got[:3], got[3].sum(axis=0, keepdims=True))
    np.testing.assert_allclose(o, o_t, atol=1e-6)  # the forward it differentiates (fp32 out)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, atol=2e-5, rtol=1e-5)


def test_backward_matches_sdpa_autograd():
    B, L, Hq, Hkv, D = 2, 16, 4, 2, 8
    q, k, v, do = rng_normal(2, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    scale = 0.3
    t = lambda x: torch.from_numpy(np.asarray(x, np.float64)).transpose(1, 2).requires_grad_(True)  # noqa: E731
    tq, tk, tv = t(q), t(k), t(v)
    o = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True, scale=scale,
                                                         enable_gqa=True)
    o.backward(torch.from_numpy(np.asarray(do, np.float64)).transpose(1, 2))
    want = [x.grad.transpose(1, 2).numpy() for x in (tq, tk, tv)]
    o_np, lse = _forward(q, k, v, mask=oracle.CausalMask(), scale=scale)
    got = attention_backward(q, k, v, o_np, do, lse, mask=oracle.CausalMask(), sm_scale=scale,
                             compute_dtype=np.float64)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, atol=2e-5, rtol=1e-5)


def _fd_check(backward_fn):
    """Central differences of L = sum(o * do) against ``backward_fn``'s gradients."""
    B, L, H, D = 1, 5, 2, 3
    q, k, v, do = (x.astype(np.float64) for x in rng_normal(3, (B, L, H, D), (B, L, H, D),
                                                             (B, L, H, D), (B, L, H, D)))
    mask = oracle.CausalMask() & oracle.KVLenMask(np.array([4], np.int32))
    scale = 0.7

    # float64 forward of the same masked softmax attention
    def loss64(q_, k_, v_):
        out = np.zeros((B, L, H, D))
        for h in range(H):
            s = q_[0, :, h] @ k_[0, :, h].T * scale
            keep = np.asarray(mask.tile_keep(0, np.arange(L), np.arange(L)), bool)
            s = np.where(keep, s, -np.inf)
            m = np.max(s, axis=-1, keepdims=True)
            p = np.exp(s - m)
            out[0, :, h] = (p / p.sum(-1, keepdims=True)) @ v_[0, :, h]
        return float(np.sum(out * do))

    o, lse = _forward(q, k, v, mask=mask, scale=scale)
    got = backward_fn(q, k, v, o.astype(np.float64), do, lse, mask=mask, sm_scale=scale,
                      compute_dtype=np.float64)
    eps = 1e-6
    worst = 0.0
    for which, x in enumerate((q, k, v)):
        num = np.zeros_like(x)
        it = np.nditer(x, flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = xp, xm
            num[idx] = (loss64(*args_p) - loss64(*args_m)) / (2 * eps)
        worst = max(worst, float(np.max(np.abs(num - got[which]))))
    return worst


def test_backward_finite_differences():
    # o from the float32-output forward differs from the float64 one by ~1e-7
    assert _fd_check(attention_backward) < 2e-5


def test_planted_missing_delta_is_rejected():
    def no_delta(q, k, v, o, do, lse, **kw):
        return attention_backward(q, k, v, np.zeros_like(o), do, lse, **kw)

    assert _fd_check(no_delta) > 1e-2


def test_closed_forms():
    B, Lq, Lk, Hq, Hkv, D = 2, 10, 12, 4, 2, 8
    q, k, v, do = rng_normal(4, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    lengths = np.array([7, 0], np.int32)  # batch 1: every row empty
    mask = oracle.KVLenMask(lengths)
    o, lse = _forward(q, k, v, mask=mask, scale=0.5)
    dq, dk, dv = attention_backward(q, k, v, o, do, lse, mask=mask, sm_scale=0.5,
                                    compute_dtype=np.float64)
    # softmax rows sum to one: sum over keys of dv = sum over queries of do (per KV head group)
    G = Hq // Hkv
    want = do[0].reshape(Lq, Hkv, G, D).sum(axis=(0, 2))
    np.testing.assert_allclose(dv[0].sum(axis=0), want, atol=1e-5)
    # masked keys and empty rows: exact zeros
    assert np.all(dk[0, 7:] == 0) and np.all(dv[0, 7:] == 0)
    assert np.all(dq[1] == 0) and np.all(dk[1] == 0) and np.all(dv[1] == 0)
    # identical keys: the scores do not depend on q's direction within a row -> dq = 0
    k_same = np.broadcast_to(k[:, :1], k.shape).copy()
    o2, lse2 = _forward(q, k_same, v, scale=0.5)
    dq2, _, _ = attention_backward(q, k_same, v, o2, do, lse2, sm_scale=0.5, compute_dtype=np.float64)
    assert np.max(np.abs(dq2)) < 1e-5


def test_preprocess_delta_is_row_dot():
    o, do = rng_normal(5, (2, 3, 4, 8), (2, 3, 4, 8))
    d = preprocess_delta(o, do)
    assert d.shape == (2, 4, 3)
    assert d[1, 2, 0] == pytest.approx(float(np.dot(o[1, 0, 2].astype(np.float64), do[1, 0, 2])), rel=1e-6)


def test_bf16_within_reference_gradient_tolerance():
    B, L, Hq, Hkv, D = 1, 64, 4, 2, 32
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(6, (B, L, Hq, D), (B, L, Hkv, D),
                                                           (B, L, Hkv, D), (B, L, Hq, D)))
    scale = 1.0 / math.sqrt(D)
    mask = oracle.CausalMask()
    o32, lse32 = _forward(q, k, v, mask=mask, scale=scale, cdt=np.float32)
    o16, lse16 = _forward(q, k, v, mask=mask, scale=scale, dtype="bf16", cdt=np.float32)
    g32 = attention_backward(q, k, v, o32, do, lse32, mask=mask, sm_scale=scale)
    g16 = attention_backward(q, k, v, o16, do, lse16, mask=mask, sm_scale=scale, dtype="bf16")
    for a, b in zip(g16, g32):
        np.testing.assert_allclose(a, b, atol=2e-2, rtol=1e-2)
    # and the bf16 casts are really applied (not a relabelled fp32 run)
    assert any(np.max(np.abs(a - b)) > 0 for a, b in zip(g16, g32))
    assert all(np.array_equal(x, oracle.round_bf16(x)) for x in g16)


def test_f16_within_tolerance_and_rounded():
    """fp16 mode: gradients within 2e-3 of fp32 (closer than bf16 mode), fp16
    valued, and really rounded (P and dS cast to fp16, not a relabelled fp32 run)."""
    B, L, Hq, Hkv, D = 1, 64, 4, 2, 32
    q, k, v, do = (oracle.round_f16(x) for x in rng_normal(6, (B, L, Hq, D), (B, L, Hkv, D),
                                                          (B, L, Hkv, D), (B, L, Hq, D)))
    scale = 1.0 / math.sqrt(D)
    mask = oracle.CausalMask()
    o32, lse32 = _forward(q, k, v, mask=mask, scale=scale, cdt=np.float32)
    oh, lseh = _forward(q, k, v, mask=mask, scale=scale, dtype="f16", cdt=np.float32)
    g32 = attention_backward(q, k, v, o32, do, lse32, mask=mask, sm_scale=scale)
    gh = attention_backward(q, k, v, oh, do, lseh, mask=mask, sm_scale=scale, dtype="f16")
    gb = attention_backward(q, k, v, o32, do, lse32, mask=mask, sm_scale=scale, dtype="bf16")
    for a, b, c in zip(gh, g32, gb):
        np.testing.assert_allclose(a, b, atol=2e-3, rtol=2e-3)
        assert np.max(np.abs(a - b)) < np.max(np.abs(c - b))
    assert any(np.max(np.abs(a - b)) > 0 for a, b in zip(gh, g32))
    assert all(np.array_equal(x, oracle.round_f16(x)) for x in gh)


@pytest.mark.parametrize("kind", ["softcap", "headscale", "alibi", "window", "segments", "prefix"])
def test_backward_with_score_modifiers_and_masks_matches_torch(kind):
    """The oracle's modifier derivatives and extended masks against torch
    float64 autograd of the same modified-score attention."""
    B, L, Hq, Hkv, D = 2, 10, 4, 2, 6
    q, k, v, do = rng_normal(7, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    scale = 0.5
    mask = bias = None
    G = Hq // Hkv
    t = lambda x: torch.from_numpy(np.asarray(x, np.float64)).requires_grad_(True)  # noqa: E731
    tq, tk, tv = t(q), t(k), t(v)
    s = torch.einsum("bqhd,bkhd->bhqk", tq, tk.repeat_interleave(G, 2)) * scale
    qi = torch.arange(L)[:, None]
    ki = torch.arange(L)[None, :]
    keep = torch.ones(B, 1, L, L, dtype=torch.bool)
    if kind == "softcap":
        bias = oracle.SoftCappingBias(1.5)
        s = 1.5 * torch.tanh(s / 1.5)
    elif kind == "headscale":
        sc = np.array([0.5, 2.0, 1.0, 3.0], np.float32)
        bias = oracle.PerHeadScaleBias(sc)
        s = s * torch.from_numpy(sc.astype(np.float64))[None, :, None, None]
    elif kind == "alibi":
        bias = oracle.SymmetricAlibiBias() + oracle.ConstantBias(0.25)
        slopes = torch.tensor([2.0 ** -(h + 1) for h in range(Hq)], dtype=torch.float64)
        s = s - slopes[None, :, None, None] * (qi - ki).abs() + 0.25
    elif kind == "window":
        mask = oracle.LocalWindowMask(3, 1) & oracle.CausalFromBottomRightMask(L, L)
        keep = keep & (((qi - ki) >= -1) & ((qi - ki) <= 3) & (qi >= ki))
    elif kind == "segments":
        ids = np.array([[0] * 4 + [1] * 6, [0] * 7 + [1] * 3], np.int32)
        mask = oracle.SameSegmentMask(ids)
        tid = torch.from_numpy(ids)
        keep = keep & (tid[:, None, :, None] == tid[:, None, None, :])
    elif kind == "prefix":
        pl = np.array([3, 0], np.int32)
        mask = oracle.PrefixLMMask(pl)
        keep = keep & ((ki[None, None] < torch.from_numpy(pl)[:, None, None, None]) | (qi >= ki))
    s = s.masked_fill(~keep, -math.inf)
    p = torch.softmax(s, -1)
    o = torch.einsum("bhqk,bkhd->bqhd", p, tv.repeat_interleave(G, 2))
    o.backward(torch.from_numpy(np.asarray(do, np.float64)))
    o_np, lse = oracle.xla_attention(q, k, v, mask=mask, bias=bias, sm_scale=scale, strategy="dense",
                                     compute_dtype=np.float64, return_lse=True)
    np.testing.assert_allclose(o_np, o.detach().numpy(), atol=1e-6)
    got = attention_backward(q, k, v, o_np, do, lse, mask=mask, bias=bias, sm_scale=scale,
                             compute_dtype=np.float64)
    for g, w in zip(got, (tq.grad, tk.grad, tv.grad)):
        np.testing.assert_allclose(g, w.numpy(), atol=2e-5, rtol=1e-5)
