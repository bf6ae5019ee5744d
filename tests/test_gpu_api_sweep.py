"""Seeded random sweep of the public API routes (``mha``, the split-KV decode
route it takes for short queries over long caches, materialised ``mla``), at
head dims that the kernels pad (any D up to 256) as well as native ones.

Bars: 16-bit output max-abs <= 2e-2 against the oracle in the same 16-bit
mode, fp32 <= 1e-5 against float64; gradients within probjax's tolerance
(tests/test_attention.py:597-626: atol 2e-2, rtol 1e-2) with atol scaled by
max(1, max|ref| / 4), fp32 gradients <= 1e-5 * max(1, max|ref|).  Every
case prints its parameters before it runs.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

TDT = {"bf16": "bfloat16", "f16": "float16", "f32": "float32"}


def _tdt(dt):
    import torch

    return getattr(torch, TDT[dt])


def _grad_check(names, got, want, low):
    for nm, g, w in zip(names, got, want):
        g = np.asarray(g, np.float64)
        w = np.asarray(w, np.float64)
        err = np.abs(g - w)
        if low:
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
        else:
            assert err.max() <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err.max():.3e}"


def _mha_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["bf16", "f16", "f32"]))
        d = int(rng.integers(1, 257))
        b, hkv = int(rng.integers(1, 3)), int(rng.choice([1, 2]))
        hq = hkv * int(rng.choice([1, 2, 4]))
        lq, lk = int(rng.integers(1, 300)), int(rng.integers(1, 400))
        if b * hq * lq * lk * max(d, 64) > 5e7:
            continue
        mask = [None, "causal", "kvlen"][int(rng.integers(3))]
        out.append((dt, b, lq, lk, hq, hkv, d, mask))
    return out


@pytest.mark.parametrize("dt,b,lq,lk,hq,hkv,d,mask", _mha_cases(40, 111))
def test_mha_any_head_dim_sweep(device, dt, b, lq, lk, hq, hkv, d, mask):
    """``mha`` with autograd at any head dim up to 256: the route zero-pads Q,
    K and V to the next kernel width (64, 128, 256), which leaves every score
    and output column unchanged, and slices the result back."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    print(f"mha {dt} B={b} Lq={lq} Lk={lk} Hq={hq} Hkv={hkv} D={d} mask={mask}", flush=True)
    q, k, v, do = rng_normal(121, (b, lq, hq, d), (b, lk, hkv, d), (b, lk, hkv, d), (b, lq, hq, d))
    low = dt != "f32"
    if low:
        q, k, v, do = (oracle.round_to(x, dt) for x in (q, k, v, do))
    am = om = None
    if mask == "causal":
        am, om = M.CausalMask(), oracle.CausalMask()
    elif mask == "kvlen":
        lens = np.random.default_rng(122).integers(0, lk + 2, size=b).astype(np.int32)
        am, om = M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)
    scale = 1.0 / math.sqrt(d)
    ts = [to_dev(x, device, _tdt(dt)).requires_grad_(True) for x in (q, k, v)]
    out = A.mha(*ts, mask=am, sm_scale=scale)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    cdt = np.float32 if low else np.float64
    o, lse = oracle.xla_attention(q, k, v, mask=om, sm_scale=scale, strategy="dense", dtype=dt, compute_dtype=cdt,
                                  return_lse=True)
    err = max_abs(to_np(out), o)
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= (2e-2 if low else 1e-5)
    want = attention_backward(q, k, v, o, do, lse, mask=om, sm_scale=scale, dtype=dt, compute_dtype=cdt)
    _grad_check(("dq", "dk", "dv"), [to_np(t.grad) for t in ts], want, low)


def _decode_route_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["bf16", "f16", "f32"]))
        d = int(rng.integers(8, 257))
        b, hkv = int(rng.integers(1, 5)), int(rng.choice([1, 2, 4, 8]))
        hq = hkv * int(rng.choice([1, 2, 4, 8]))
        lq = int(rng.integers(1, 9))
        lk = int(rng.integers(1024, 3000))
        if b * hq * lq * lk * max(d, 64) > 2e8:
            continue
        lengths = bool(rng.random() < 0.6)
        out.append((dt, b, lq, lk, hq, hkv, d, lengths))
    return out


@pytest.mark.parametrize("dt,b,lq,lk,hq,hkv,d,lengths", _decode_route_cases(24, 131))
def test_mha_decode_route_sweep(device, dt, b, lq, lk, hq, hkv, d, lengths):
    """Short queries over caches of >= 1024 keys, without a mask or with a
    KVLenMask: ``mha`` takes the split-KV decode (probjax's rule, Lq <= 64 and
    Lkv >= 1024), at any head dim up to 256 (padded), against the oracle."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M
    from probjax_amd import native

    print(f"decode route {dt} B={b} Lq={lq} Lk={lk} Hq={hq} Hkv={hkv} D={d} lengths={lengths}", flush=True)
    q, k, v = rng_normal(141, (b, lq, hq, d), (b, lk, hkv, d), (b, lk, hkv, d))
    low = dt != "f32"
    if low:
        q, k, v = (oracle.round_to(x, dt) for x in (q, k, v))
    am = om = None
    if lengths:
        lens = np.random.default_rng(142).integers(0, lk + 2, size=b).astype(np.int32)
        am, om = M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)
    scale = 1.0 / math.sqrt(d)
    with torch.no_grad():
        out = A.mha(*(to_dev(x, device, _tdt(dt)) for x in (q, k, v)), mask=am, sm_scale=scale)
    launched = native.last_launches()
    torch.cuda.synchronize()
    assert A.use_splitkv(to_dev(q, device, _tdt(dt)), to_dev(k, device, _tdt(dt)), mask=am)
    assert any(n.startswith("gqa_decode") for n in launched), launched
    want = oracle.xla_attention(q, k, v, mask=om, sm_scale=scale, strategy="dense", dtype=dt,
                                compute_dtype=np.float32 if low else np.float64)
    err = max_abs(to_np(out), want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= (2e-2 if low else 1e-5)


def _mla_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["bf16", "f16", "f32"]))
        b, h = int(rng.integers(1, 3)), int(rng.integers(1, 5))
        lq, s = int(rng.integers(2, 200)), int(rng.integers(2, 260))
        r = int(rng.integers(8, 300))
        dk, dv = int(rng.integers(8, 257)), int(rng.integers(8, 257))
        if b * h * lq * s * max(dk, dv, 64) > 3e7:
            continue
        causal = bool(rng.random() < 0.5)
        out.append((dt, b, lq, s, h, r, dk, dv, causal))
    return out


@pytest.mark.parametrize("dt,b,lq,s,h,r,dk,dv,causal", _mla_cases(20, 151))
def test_materialized_mla_sweep(device, dt, b, lq, s, h, r, dk, dv, causal):
    """``mla(q, cache, wk, wv)`` with gradients for all four inputs, any rank
    and head dims (the projection kernel pads K and V to the flash width),
    against the oracle's materialised computation and its VJP."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    print(f"mla-mat {dt} B={b} Lq={lq} S={s} H={h} R={r} dk={dk} dv={dv} causal={causal}", flush=True)
    q, cache, do = rng_normal(161, (b, lq, h, dk), (b, s, r), (b, lq, h, dv))
    wk, wv = rng_normal(162, (h, dk, r), (h, dv, r), scale=1 / math.sqrt(r))
    low = dt != "f32"
    if low:
        q, cache, wk, wv, do = (oracle.round_to(x, dt) for x in (q, cache, wk, wv, do))
    am, om = (M.CausalMask(), oracle.CausalMask()) if causal else (None, None)
    ts = [to_dev(x, device, _tdt(dt)).requires_grad_(True) for x in (q, cache, wk, wv)]
    out = A.mla(*ts, mask=am)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    kw = dict(mask=om, dtype=dt, compute_dtype=np.float32 if low else np.float64)
    o_want = oracle.materialized_mla(q, cache, wk, wv, **kw)
    err = max_abs(to_np(out), o_want)
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= (2e-2 if low else 1e-5)
    got = [to_np(t.grad) for t in ts]
    if not low:
        want = oracle.materialized_mla_backward(q, cache, wk, wv, do, **kw)
        _grad_check(("dq", "dcache", "dwk", "dwv"), got, want, low)
        return
    # 16-bit: the weight gradients sum dK / dV (each carrying the roundings
    # of P and dS) against C over every key, so two independent sets of
    # roundings can differ by more than one 16-bit step there.  The kernel
    # and the oracle's own 16-bit mode are therefore both compared with the
    # exact (float64) gradient: max error within probjax's tolerance (or
    # within 1.5x the oracle's own, where that exceeds it), and an
    # RMS error at most 1.5x the oracle's plus 2^-10 of the gradient's scale
    # (rows that see one or two keys carry pure rounding noise, which over a
    # few dozen values makes the RMS ratio itself noisy).
    exact = oracle.materialized_mla_backward(q, cache, wk, wv, do, mask=om, dtype="f32", compute_dtype=np.float64)
    mode = oracle.materialized_mla_backward(q, cache, wk, wv, do, **kw)
    for nm, g, e, m in zip(("dq", "dcache", "dwk", "dwv"), got, exact, mode):
        g, e, m = (np.asarray(x, np.float64) for x in (g, e, m))
        scale_w = max(1.0, float(np.max(np.abs(e))))
        err, err_ref = np.abs(g - e), np.abs(m - e)
        within = (err <= 2e-2 * max(1.0, scale_w / 4.0) + 1e-2 * np.abs(e)).all()
        # where the oracle's own 16-bit arithmetic already exceeds that bar
        # (small weight gradients summed over few keys), no worse than 1.5x it
        assert within or err.max() <= 1.5 * err_ref.max(), f"{nm}: max err {err.max():.3e} ({err_ref.max():.3e})"
        rms, rms_ref = float(np.sqrt(np.mean(err ** 2))), float(np.sqrt(np.mean(err_ref ** 2)))
        print(f"  {nm}: max err {err.max():.3e}, rms {rms:.3e} (16-bit oracle rms {rms_ref:.3e})", flush=True)
        assert rms <= 1.5 * rms_ref + 2.0 ** -10 * scale_w, f"{nm}: rms {rms:.3e} against {rms_ref:.3e}"
