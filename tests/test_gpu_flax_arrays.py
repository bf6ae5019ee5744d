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

from tests._helpers import rng_normal, to_dev, to_np

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
