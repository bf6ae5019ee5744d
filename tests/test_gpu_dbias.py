"""Gradient of a dense bias on the GPU.

``dot_product_attention`` gives a ``DenseBias`` tensor that requires grad its
gradient, as probjax's dense path does (autodiff of ``scores + bias``,
layers/attention.py:1293-1319): ``P (dP - delta)`` per score, summed over the
dimensions the bias broadcasts.  ``flex_attention`` keeps the reference
kernel VJP's zero cotangent for bias data (kernels/attention.py:3262-3263).

Tolerances: against ``oracle.attention_backward(return_dbias=True)`` on the
oracle forward's output and LSE; bf16 within probjax's gradient tolerance
(atol 2e-2 scaled by max(1, max|ref| / 4), rtol 1e-2), fp32 max-abs
<= 1e-5 * max(1, max|ref|) against the float64 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

CASES = [
    # dtype, B, L, Hq, Hkv, D, bias batch, bias heads, mask, alibi
    ("bf16", 2, 256, 4, 2, 128, 1, 4, "causal", False),
    ("bf16", 2, 200, 2, 2, 64, 2, 1, "kvlen", False),
    ("bf16", 1, 192, 4, 4, 64, 1, 1, "causal", True),   # dense bias + ALiBi (full extended path)
    ("f32", 2, 130, 2, 1, 64, 2, 2, "kvlen", False),
    ("f32", 1, 96, 2, 2, 128, 1, 2, "causal", True),
]


@pytest.mark.parametrize("dtype,B,L,Hq,Hkv,D,bb,bh,mask_name,alibi", CASES)
def test_dense_bias_gradient(device, dtype, B, L, Hq, Hkv, D, bb, bh, mask_name, alibi):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    print(f"dbias {dtype} B={B} L={L} Hq={Hq} Hkv={Hkv} D={D} bias=[{bb},{bh}] {mask_name} alibi={alibi}",
          flush=True)
    q, k, v, do = rng_normal(80, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    (bias,) = rng_normal(81, (bb, bh, L, L), scale=0.5)
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    lens = np.array([L, L // 3][:B], np.int32)
    if mask_name == "causal":
        mask, omask = M.CausalMask(), oracle.CausalMask()
    else:
        mask, omask = M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)
    tb = to_dev(bias, device, torch.float32).requires_grad_(True)
    mbias, obias = M.DenseBias(tb), oracle.DenseBias(bias)
    if alibi:
        mbias, obias = mbias + M.CausalAlibiBias(), obias + oracle.CausalAlibiBias()
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.dot_product_attention(tq, tk, tv, mask=mask, bias=mbias)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    assert tb.grad is not None and tb.grad.shape == (bb, bh, L, L)
    scale = 1.0 / math.sqrt(D)
    cdt = np.float32 if bf16 else np.float64
    o, lse = oracle.xla_attention(q, k, v, mask=omask, bias=obias, sm_scale=scale, strategy="dense",
                                  dtype=dtype, compute_dtype=cdt, return_lse=True)
    *grads, dbias = attention_backward(q, k, v, o, do, lse, mask=omask, bias=obias, sm_scale=scale,
                                       dtype=dtype, compute_dtype=cdt, return_dbias=True)
    dims = tuple(d for d, n in ((0, bb), (1, bh)) if n == 1)
    want_db = dbias.sum(axis=dims, keepdims=True) if dims else dbias
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv, tb)]
    want = [*grads, want_db]
    if bf16:
        assert max_abs(to_np(out), o) <= 2e-2
        for nm, g, w in zip(("dq", "dk", "dv", "dbias"), got, want):
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(to_np(out), o) <= 1e-5
        for nm, g, w in zip(("dq", "dk", "dv", "dbias"), got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"
    # masked scores get exactly zero gradient
    keep = np.stack([omask.tile_keep(b, np.arange(L), np.arange(L)) for b in range(B)])
    if bb == B:
        assert not np.any(got[3][np.broadcast_to(~keep[:, None], got[3].shape)])

    # flex_attention: the reference kernel path's zero cotangent for bias data
    tb2 = to_dev(bias, device, torch.float32).requires_grad_(True)
    tq2 = to_dev(q, device, tdt).requires_grad_(True)
    out2 = A.flex_attention(tq2, to_dev(k, device, tdt), to_dev(v, device, tdt), mask=mask,
                            bias=M.DenseBias(tb2), enable_gqa=Hq != Hkv)
    out2.float().sum().backward()
    assert tb2.grad is None and tq2.grad is not None
