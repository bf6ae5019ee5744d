"""Masks and biases without an in-kernel form on the GPU: NOT / OR / XOR
compositions, MarginalizationMask, and T5 / learned relative-position
tables.  The route lowers them to a dense additive fp32 bias (0 / -inf for a
mask, the table gathered per (q, k) for a relative-position term) on the
flash kernels; gradients reach a relative-position table through
``dot_product_attention`` (probjax's dense path).  Against the oracle's
evaluation of the same objects.

Tolerances: bf16 output max-abs <= 2e-2 against the fp32 oracle from the same
bf16-rounded inputs, gradients within probjax's gradient tolerance (atol
2e-2 scaled by max(1, max|ref| / 4), rtol 1e-2); fp32 output <= 1e-5 and
gradients <= 1e-5 * max(1, max|ref|) against the float64 oracle.

The bf16 relative-position gradients are referenced to the oracle backward of
the kernel's own bf16 forward output (the output the kernel backward receives, as
in autograd): the learned table's far bucket sums dL/d(bias) = P (dP - delta)
over most of the causal triangle, and one-ulp differences between two
correctly rounded bf16 outputs move delta, and that sum, by more than the
tolerance.  The output itself is checked against the oracle's.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _masks(name, B, L, dev):
    import torch
    from probjax_amd import masks as M

    rng = np.random.default_rng(90)
    marg = rng.random((B, L)) < 0.5
    lens = np.array([L, L // 2][:B], np.int32)
    tm, tl = torch.from_numpy(marg).to(dev), torch.from_numpy(lens).to(dev)
    return {
        "or": (M.CausalMask() | M.LocalWindowMask(16, 40), oracle.CausalMask() | oracle.LocalWindowMask(16, 40)),
        "not": (~M.LocalWindowMask(8, 8), ~oracle.LocalWindowMask(8, 8)),
        "xor_kvlen": (M.CausalMask() ^ M.KVLenMask(tl), oracle.CausalMask() ^ oracle.KVLenMask(lens)),
        "marginalization": (M.MarginalizationMask(tm), oracle.MarginalizationMask(marg)),
        "marg_causal": (M.MarginalizationMask(tm) & M.CausalMask(), oracle.MarginalizationMask(marg) & oracle.CausalMask()),
    }[name]


CASES = [
    ("or", "bf16", 2, 256, 4, 2, 128),
    ("not", "bf16", 1, 200, 2, 2, 64),
    ("xor_kvlen", "bf16", 2, 192, 4, 4, 64),
    ("marginalization", "bf16", 2, 160, 2, 1, 128),
    ("marg_causal", "f32", 2, 128, 2, 2, 64),
    ("or", "f32", 1, 96, 2, 2, 128),
]


def _check(dtype, got_o, want_o, got, want, names):
    if dtype == "bf16":
        assert max_abs(got_o, want_o) <= 2e-2
        for nm, g, w in zip(names, got, want):
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(got_o, want_o) <= 1e-5
        for nm, g, w in zip(names, got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"


@pytest.mark.parametrize("name,dtype,B,L,Hq,Hkv,D", CASES)
def test_dense_lowered_masks(device, name, dtype, B, L, Hq, Hkv, D):
    import torch
    from probjax_amd import attention as A

    print(f"dense mask {name} {dtype} B={B} L={L} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    q, k, v, do = rng_normal(91, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    mask, omask = _masks(name, B, L, device)
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.flex_attention(tq, tk, tv, mask=mask, enable_gqa=Hq != Hkv)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    cdt = np.float32 if bf16 else np.float64
    o, lse = oracle.xla_attention(q, k, v, mask=omask, sm_scale=scale, strategy="dense", dtype=dtype,
                                  compute_dtype=cdt, return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=omask, sm_scale=scale, dtype=dtype, compute_dtype=cdt)
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv)]
    _check(dtype, to_np(out), o, got, want, ("dq", "dk", "dv"))


@pytest.mark.parametrize("kind,dtype", [("t5", "bf16"), ("t5_uni", "f32"), ("learned", "bf16")])
def test_relative_position_tables(device, kind, dtype):
    """dot_product_attention gives the table its gradient (the sum of dL/d(bias)
    over the (q, k) pairs of each bucket); flex_attention gives it none."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    B, L, H, D = 2, 160, 4, 64
    print(f"relpos {kind} {dtype} B={B} L={L} H={H} D={D}", flush=True)
    q, k, v, do = rng_normal(92, (B, L, H, D), (B, L, H, D), (B, L, H, D), (B, L, H, D))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    rel = np.arange(L)[None, :] - np.arange(L)[:, None]
    if kind.startswith("t5"):
        bi = kind == "t5"
        table = rng_normal(93, (H, 32))[0]
        obias = oracle.T5RelativePositionBias(table, num_buckets=32, max_distance=64, bidirectional=bi)
        tt = to_dev(table, device, torch.float32).requires_grad_(True)
        mbias = M.T5RelativePositionBias(tt, num_buckets=32, max_distance=64, bidirectional=bi)
        idx = oracle.masks.relative_position_bucket(rel, num_buckets=32, max_distance=64, bidirectional=bi)
    else:
        table = rng_normal(94, (1, 2 * 20 + 1))[0]
        obias = oracle.LearnedRelativePositionBias(table, max_distance=20)
        tt = to_dev(table, device, torch.float32).requires_grad_(True)
        mbias = M.LearnedRelativePositionBias(tt, max_distance=20)
        idx = np.clip(rel, -20, 20) + 20
    mask, omask = M.CausalMask(), oracle.CausalMask()
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.dot_product_attention(tq, tk, tv, mask=mask, bias=mbias)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    cdt = np.float32 if bf16 else np.float64
    o, lse = oracle.xla_attention(q, k, v, mask=omask, bias=obias, sm_scale=scale, strategy="dense",
                                  dtype=dtype, compute_dtype=cdt, return_lse=True)
    o_bwd = to_np(out).astype(np.float32) if bf16 else o
    *want, dbias = attention_backward(q, k, v, o_bwd, do, lse, mask=omask, bias=obias, sm_scale=scale,
                                      dtype=dtype, compute_dtype=cdt, return_dbias=True)
    dtable = np.zeros(table.shape, np.float64)
    per_head = dbias.sum(axis=0)  # [H, L, L]
    for h in range(H):
        np.add.at(dtable[h if table.shape[0] > 1 else 0], idx, per_head[h])
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv, tt)]
    _check(dtype, to_np(out), o, got, [*want, dtable], ("dq", "dk", "dv", "dtable"))
    # flex_attention: the reference kernel VJP's zero cotangent for bias data
    tt2 = to_dev(table, device, torch.float32).requires_grad_(True)
    b2 = (M.T5RelativePositionBias(tt2, num_buckets=32, max_distance=64, bidirectional=kind == "t5")
          if kind.startswith("t5") else M.LearnedRelativePositionBias(tt2, max_distance=20))
    tq2 = to_dev(q, device, tdt).requires_grad_(True)
    A.flex_attention(tq2, to_dev(k, device, tdt), to_dev(v, device, tdt), mask=mask, bias=b2).float().sum().backward()
    assert tt2.grad is None and tq2.grad is not None
