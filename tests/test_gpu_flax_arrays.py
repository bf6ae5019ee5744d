"""Flax-style array masks and biases through ``dot_product_attention`` on the
GPU.  probjax hands arrays to ``flax.linen.dot_product_attention``
(layers/attention.py:1298-1319): scores ``q.k / sqrt(D) + bias``, masked
scores replaced by the dtype's most negative value, softmax, weights cast to
the value dtype, then ``weights . v``.  A row whose keys are all masked
therefore gets equal weights over every key.  The reference here is that
computation in torch on the CPU (float32 for bf16 inputs, float64 for fp32),
with autograd for the gradients; the mirror lowers the arrays to a dense
additive bias on the flash kernels and fills fully masked rows with the mean
of V.

Tolerances: bf16 output max-abs <= 2e-2, gradients within probjax's gradient
tolerance (atol 2e-2 scaled by max(1, max|ref| / 4), rtol 1e-2); fp32 output
<= 1e-5 and gradients <= 1e-5 * max(1, max|ref|).
"""

import math

import numpy as np
import pytest

from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _flax_reference(q, k, v, mask, bias, wdtype):
    """Flax dot_product_attention on [..., L, H, D] tensors (GQA by repeating
    K/V heads); mask/bias broadcast to [..., H, Lq, Lk]."""
    import torch

    g = q.shape[-2] // k.shape[-2]
    k = k.repeat_interleave(g, dim=-2)
    v = v.repeat_interleave(g, dim=-2)
    s = torch.einsum("...qhd,...khd->...hqk", q / math.sqrt(q.shape[-1]), k)
    if bias is not None:
        s = s + bias
    if mask is not None:
        s = torch.where(mask, s, torch.tensor(torch.finfo(torch.float32).min, dtype=s.dtype))
    w = torch.softmax(s, dim=-1)
    if wdtype is not None:
        w = w.to(wdtype).to(s.dtype)
    return torch.einsum("...hqk,...khd->...qhd", w, v)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_array_mask_and_bias(device, dtype):
    import torch
    from probjax_amd import attention as A

    bf16 = dtype == "bf16"
    lead, L, Hq, Hkv, D = (2, 3), 96, 4, 2, 64
    print(f"flax arrays {dtype} lead={lead} L={L} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    q, k, v, do = rng_normal(120, lead + (L, Hq, D), lead + (L, Hkv, D), lead + (L, Hkv, D), lead + (L, Hq, D))
    (bias,) = rng_normal(121, (Hq, L, L), scale=0.5)
    keep = np.random.default_rng(122).random((3, 1, L, L)) < 0.8
    keep[1, 0, 5] = False  # one row of the second batch column drops every key
    tdt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    tb = to_dev(bias, device, torch.float32).requires_grad_(True)
    tm = torch.from_numpy(keep).to(device)
    out = A.dot_product_attention(tq, tk, tv, mask=tm, bias=tb)
    assert out.shape == lead + (L, Hq, D)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    cdt = torch.float32 if bf16 else torch.float64
    rq, rk, rv = (torch.from_numpy(np.asarray(to_np(t), np.float64)).to(cdt).requires_grad_(True) for t in (tq, tk, tv))
    rb = torch.from_numpy(bias.astype(np.float64)).to(cdt).requires_grad_(True)
    ro = _flax_reference(rq, rk, rv, torch.from_numpy(keep), rb, torch.bfloat16 if bf16 else None)
    (ro * torch.from_numpy(do.astype(np.float64)).to(cdt)).sum().backward()

    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv, tb)]
    want = [t.grad.double().numpy() for t in (rq, rk, rv, rb)]
    o_err = float(np.max(np.abs(to_np(out) - ro.detach().double().numpy())))
    # the fully masked row is the mean of V over every key
    vm = to_np(tv)[1, :, :, :, :].mean(axis=1)  # [3, Hkv, D] (batch column 1 holds index 1)
    np.testing.assert_allclose(to_np(out)[1, 1, 5], np.repeat(vm[1], Hq // Hkv, axis=0), atol=2e-2 if bf16 else 1e-5)
    if bf16:
        assert o_err <= 2e-2
        for nm, g, w in zip(("dq", "dk", "dv", "dbias"), got, want):
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert o_err <= 1e-5
        for nm, g, w in zip(("dq", "dk", "dv", "dbias"), got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"


def _alibi_dense(Hq, Lq, Lk):
    """CausalAlibiBias as a dense [Hq, Lq, Lk] bias: -2^-(h+1) * max(q - k, 0)
    (attention_mask_bias.py:2230-2255)."""
    d = np.maximum(np.arange(Lq)[:, None] - np.arange(Lk)[None, :], 0).astype(np.float64)
    return np.stack([-(2.0 ** -(h + 1.0)) * d for h in range(Hq)])


# (name, Lq, Lk, Hq, Hkv, D, mask kind, bias kind)
_CASES = [
    ("mask_only_per_head", 80, 112, 4, 4, 64, "array_per_head", None),
    ("bias_only_d128", 64, 96, 4, 2, 128, None, "array"),
    ("array_mask_object_alibi", 72, 72, 4, 2, 64, "array", "alibi"),
    ("kvlen_zero_array_bias", 48, 80, 4, 2, 64, "kvlen0", "array"),
    ("kvlen_zero_dense_object", 48, 80, 2, 1, 128, "kvlen0", "dense_object"),
    ("padded_d96", 64, 64, 2, 2, 96, "array", "array"),
    # no bias: KVLenMask is not one of probjax's fused masks, so Flax's einsum
    ("kvlen_zero_no_bias", 48, 80, 4, 2, 64, "kvlen0", None),
    # a fused mask type under 64 keys: Flax's einsum too (rows 42.. keep no key)
    ("window_short_keys", 48, 40, 4, 4, 64, "window2", None),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("case", _CASES, ids=[c[0] for c in _CASES])
def test_flax_semantics_cases(device, dtype, case):
    """Array masks alone, biases alone, Lq != Lk, per-head masks, an object
    bias with an array mask, and object masks whose rows drop every key
    (KVLenMask with a zero length, with and without a bias; a local window
    over fewer than 64 keys): wherever probjax takes the Flax einsum (a bias,
    an array mask, a mask outside its fused set, fewer than 64 keys), such
    rows are the mean of V, with dV = dO / Lk and no gradient to q, k or the
    bias there."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    name, Lq, Lk, Hq, Hkv, D, mkind, bkind = case
    bf16 = dtype == "bf16"
    B = 3
    print(f"flax case {name} {dtype}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    seed = 130 + _CASES.index(case)
    q, k, v, do = rng_normal(seed, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    rng = np.random.default_rng(seed + 1000)
    tdt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    keep = None
    mask_arg = None
    if mkind == "array":
        keep = rng.random((B, 1, Lq, Lk)) < 0.8
        keep[1, 0, 3] = False
        mask_arg = torch.from_numpy(keep).to(device)
    elif mkind == "array_per_head":
        keep = rng.random((Hq, Lq, Lk)) < 0.75
        keep[2, 7] = False
        mask_arg = torch.from_numpy(keep).to(device)
        keep = np.broadcast_to(keep[None], (B, Hq, Lq, Lk))
    elif mkind == "kvlen0":
        lengths = np.array([Lk, 0, Lk - 17], np.int32)
        keep = np.broadcast_to((np.arange(Lk)[None, :] < lengths[:, None])[:, None, None, :], (B, 1, Lq, Lk))
        mask_arg = M.KVLenMask(torch.from_numpy(lengths).to(device))
    elif mkind == "window2":
        d = np.arange(Lq)[:, None] - np.arange(Lk)[None, :]
        keep = np.broadcast_to(((d >= 0) & (d <= 2))[None, None], (B, 1, Lq, Lk))
        assert not keep[0, 0, -1].any()  # the last rows keep no key
        mask_arg = M.LocalWindowMask(2, 0)
    bias_ref = None
    bias_arg = None
    tb = None
    if bkind == "array":
        (bias,) = rng_normal(seed + 2000, (Hq, Lq, Lk), scale=0.5)
        tb = to_dev(bias, device, torch.float32).requires_grad_(True)
        bias_arg, bias_ref = tb, bias.astype(np.float64)
    elif bkind == "dense_object":
        (bias,) = rng_normal(seed + 2000, (B, Hq, Lq, Lk), scale=0.5)
        tb = to_dev(bias, device, torch.float32).requires_grad_(True)
        bias_arg, bias_ref = M.DenseBias(tb), bias.astype(np.float64)
    elif bkind == "alibi":
        bias_arg, bias_ref = M.CausalAlibiBias(), _alibi_dense(Hq, Lq, Lk)

    out = A.dot_product_attention(tq, tk, tv, mask=mask_arg, bias=bias_arg)
    assert out.shape == (B, Lq, Hq, D)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    cdt = torch.float32 if bf16 else torch.float64
    rq, rk, rv = (torch.from_numpy(np.asarray(to_np(t), np.float64)).to(cdt).requires_grad_(True) for t in (tq, tk, tv))
    rb = None
    if bias_ref is not None:
        rb = torch.from_numpy(np.ascontiguousarray(bias_ref)).to(cdt).requires_grad_(tb is not None)
    rm = None if keep is None else torch.from_numpy(np.ascontiguousarray(keep))
    ro = _flax_reference(rq, rk, rv, rm, rb, torch.bfloat16 if bf16 else None)
    (ro * torch.from_numpy(do.astype(np.float64)).to(cdt)).sum().backward()

    got_o = to_np(out).astype(np.float64)
    want_o = ro.detach().double().numpy()
    pairs = [("dq", tq, rq), ("dk", tk, rk), ("dv", tv, rv)]
    if tb is not None:
        pairs.append(("dbias", tb, rb))
    if bf16:
        assert max_abs(got_o, want_o) <= 2e-2, f"out: {max_abs(got_o, want_o):.3e}"
        for nm, g, w in pairs:
            g, w = to_np(g.grad).astype(np.float64), w.grad.double().numpy()
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(got_o, want_o) <= 1e-5, f"out: {max_abs(got_o, want_o):.3e}"
        for nm, g, w in pairs:
            g, w = to_np(g.grad).astype(np.float64), w.grad.double().numpy()
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"
