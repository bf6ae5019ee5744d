"""Low-rank and learned-ALiBi biases through ``flex_attention`` on the GPU:
the factors are folded into Q/K (probjax layers/attention.py:1600-1635) and
the flash kernels run on the folded inputs; gradients reach q, k, v and the
factor tensors through torch autograd.  Against ``oracle.flex_low_rank`` and
its VJP.

Tolerances: bf16 output max-abs <= 2e-2 against the fp32 oracle from the same
bf16-rounded inputs, gradients within probjax's gradient tolerance (atol
2e-2, rtol 1e-2, tests/test_attention.py:597-626) with atol scaled by
max(1, max|ref| / 4), and by 3 more for the factor gradients (two extra bf16
roundings on their way from the folded features); fp32
output <= 1e-5 and gradients <= 1e-5 * max(1, max|ref|) against the float64
oracle.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.lowrank import flex_low_rank, flex_low_rank_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _case(name, B, L, Hq, dev):
    """(mirror bias, oracle bias, factor arrays, causal)."""
    import torch
    from probjax_amd import masks as M

    if name in ("low_rank", "sum"):
        qf, kf = rng_normal(70, (Hq, L + 20, 8), (Hq, L + 20, 8))
        t = [to_dev(x, dev, torch.float32).requires_grad_(True) for x in (qf, kf)]
        mine, theirs = M.LowRankBias(*t, scale=0.5), oracle.LowRankBias(qf, kf, scale=0.5)
        if name == "sum":
            mine, theirs = mine + M.CausalAlibiBias(), theirs + oracle.CausalAlibiBias()
        return mine, theirs, t, name == "sum"
    if name == "shared":
        # scale 0.75: a fold scale near 4 makes the softmax so peaked that dS =
        # P (dP - delta) cancels almost exactly, and one-ulp differences of the
        # bf16 forward output move delta by more than the gradient tolerance
        qf, kf = rng_normal(71, (1, L, 4), (1, L, 4))
        t = [to_dev(x, dev, torch.float32).requires_grad_(True) for x in (qf, kf)]
        return M.LowRankBias(*t, scale=0.75), oracle.LowRankBias(qf, kf, scale=0.75), t, False
    if name == "key_bias":
        (kb,) = rng_normal(72, (B, L))
        tk = to_dev(kb, dev, torch.float32).requires_grad_(True)
        mine = M.BatchedLowRankBias.from_key_bias(tk)
        theirs = oracle.BatchedLowRankBias.from_key_bias(kb)
        return mine, theirs, [tk], True
    if name == "alibi":
        log_slopes = np.log(np.array([0.5, 0.25, 0.125, 0.0625][:Hq], np.float32))
        tl = to_dev(log_slopes, dev, torch.float32).requires_grad_(True)
        return (M.LearnedAlibiBias(torch.exp(tl)), oracle.LearnedAlibiBias(np.exp(log_slopes)), [tl], True)
    raise KeyError(name)


CASES = [
    # name, dtype, B, L, Hq, Hkv, D
    ("low_rank", "bf16", 2, 256, 4, 2, 64),
    ("low_rank", "f32", 1, 128, 2, 2, 64),
    ("shared", "bf16", 1, 200, 2, 1, 96),
    ("key_bias", "bf16", 2, 192, 2, 2, 64),
    ("alibi", "bf16", 1, 256, 4, 4, 64),
    ("alibi", "f32", 1, 96, 4, 2, 32),
    ("sum", "bf16", 2, 160, 4, 4, 64),
]


@pytest.mark.parametrize("name,dtype,B,L,Hq,Hkv,D", CASES)
def test_low_rank_bias_forward_and_grads(device, name, dtype, B, L, Hq, Hkv, D):
    import torch
    from probjax_amd import attention as A

    print(f"low-rank {name} {dtype} B={B} L={L} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    q, k, v, do = rng_normal(73, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    mine, theirs, factors, causal = _case(name, B, L, Hq, device)
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    mask = None
    if causal:
        from probjax_amd.masks import CausalMask

        mask = CausalMask()
    out = A.flex_attention(tq, tk, tv, mask=mask, bias=mine, enable_gqa=Hq != Hkv)
    assert out.shape == (B, L, Hq, D)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    scale = 1 / math.sqrt(D)
    omask = oracle.CausalMask() if causal else None
    cdt = np.float32 if bf16 else np.float64
    kw = dict(mask=omask, bias=theirs, sm_scale=scale, dtype=dtype, compute_dtype=cdt)
    o_want = flex_low_rank(q, k, v, **kw)
    dq, dk, dv, fg, feats = flex_low_rank_backward(q, k, v, do, return_features=True, **kw)
    want = [dq, dk, dv, *fg[0]]
    slope_atol = None
    if name == "alibi":
        # the leaf is log(slopes): d/dlog s = s * d/ds
        s_ = np.exp(to_np(factors[0]).astype(np.float64))
        want[3] = want[3] * s_
        # d/ds = sum_q gq[q, 0] * (-q) + sum_k gk[k, 1] * k: sums of positions
        # times bf16 feature cotangents that cancel; each term carries ~1 bf16
        # rounding step, so the bound is 2^-7 of the summed term magnitudes.
        gq, gk = feats[0]
        pos = np.arange(L, dtype=np.float64)
        mag = np.einsum("bqh,q->h", np.abs(gq[..., 0]), pos) + np.einsum("bkh,k->h", np.abs(gk[..., 1]), pos)
        slope_atol = 2.0 ** -7 * mag * s_
    if name == "key_bias":
        # the leaf is key_bias [B, L]: the key factors are key_bias[..., None]
        want = [dq, dk, dv, fg[0][1][..., 0]]
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv, *factors)]
    names = ["dq", "dk", "dv"] + [f"dfactor{i}" for i in range(len(factors))]
    if bf16:
        assert max_abs(to_np(out), o_want) <= 2e-2
        for i, (nm, g, w) in enumerate(zip(names, got, want)):
            # A factor gradient passes two more bf16 roundings than dq / dk
            # (the folded feature's gradient dq' is rounded, then multiplied by
            # the fold scale and rounded again) before the sums over heads or
            # batch: 3x the base bound.
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0) * (3.0 if i >= 3 else 1.0)
            if i == 3 and slope_atol is not None:
                atol = np.maximum(atol, slope_atol)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(to_np(out), o_want) <= 1e-5
        for nm, g, w in zip(names, got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"
    if name == "alibi":
        assert np.all(np.isfinite(got[3])) and np.any(got[3] != 0)
