"""Seeded random-shape parity sweep over every kernel family.

The hand-picked cases of the other files pin each launcher branch; this file
draws shapes from a fixed generator (batch, heads, GQA group, ragged query and
key lengths, head dims 64 / 128 / 256, dtype, causal, key lengths past or
below the capacity, broadcast dense biases, decode row counts and chunk
sizes, latent ranks) so that combinations nobody wrote down also meet the bar
against the CPU oracle:

* forward: fp32 max-abs <= 1e-5 against the float64 oracle; bf16 / fp16
  max-abs <= 2e-2 against the oracle in the same 16-bit mode (P rounded before
  P.V, attention_xla.py:349); rows without a valid key exactly 0, LSE +inf;
* backward: probjax's gradient tolerance (tests/test_attention.py:597-626:
  atol 2e-2, rtol 1e-2) in 16-bit, 1e-5 * max(1, max|ref|) in fp32 against
  float64; keys past their length get exactly zero dK / dV;
* split-KV decode and latent decode / prefill: as the forward.

Every case prints its parameters before it runs.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
HALF_TOL = 2e-2
ATOL, RTOL = 2e-2, 1e-2


def _tdt(dt):
    import torch

    return {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]


def _mask(causal, lengths):
    m = oracle.CausalMask() if causal else None
    if lengths is not None:
        kl = oracle.KVLenMask(np.array(lengths, np.int32))
        m = kl if m is None else m & kl
    return m


def _flash_cases(n, seed, budget):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["f32", "bf16", "f16"]))
        d = int(rng.choice([64, 128, 256]))
        b = int(rng.integers(1, 4))
        hkv = int(rng.choice([1, 2, 3]))
        hq = hkv * int(rng.choice([1, 2, 4]))
        lq, lk = int(rng.integers(1, 640)), int(rng.integers(1, 900))
        if b * hq * lq * lk * d > budget:
            continue
        causal = bool(rng.random() < 0.5)
        lengths = [int(x) for x in rng.integers(-2, lk + 4, size=b)] if rng.random() < 0.4 else None
        bias = (int(rng.choice([1, b])), int(rng.choice([1, hq]))) if rng.random() < 0.3 else None
        out.append((dt, b, lq, lk, hq, hkv, d, causal, lengths, bias))
    return out


def _inputs(seed, dt, b, lq, lk, hq, hkv, d, bias_shape):
    q, k, v, do = rng_normal(seed, (b, lq, hq, d), (b, lk, hkv, d), (b, lk, hkv, d), (b, lq, hq, d))
    if dt != "f32":
        q, k, v, do = (oracle.round_to(x, dt) for x in (q, k, v, do))
    bias = None if bias_shape is None else rng_normal(seed + 1, (*bias_shape, lq, lk), scale=0.5)[0]
    return q, k, v, do, bias


FWD_CASES = _flash_cases(96, 2026, 3e8)


@pytest.mark.parametrize("dt,b,lq,lk,hq,hkv,d,causal,lengths,bias_shape", FWD_CASES)
def test_forward_sweep(device, dt, b, lq, lk, hq, hkv, d, causal, lengths, bias_shape):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    print(f"fwd {dt} B={b} Lq={lq} Lk={lk} Hq={hq} Hkv={hkv} D={d} causal={causal} "
          f"lengths={lengths} bias={bias_shape}", flush=True)
    q, k, v, _, bias = _inputs(101, dt, b, lq, lk, hq, hkv, d, bias_shape)
    scale = 1.0 / math.sqrt(d)
    mask = _mask(causal, lengths)
    db = None if bias is None else oracle.DenseBias(bias)
    f32 = dt == "f32"
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, bias=db, sm_scale=scale, strategy="dense",
                                          dtype=dt, compute_dtype=np.float64 if f32 else np.float32,
                                          return_lse=True)
    t = _tdt(dt)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got, lse = flash_attention_fwd(*(to_dev(x, device, t) for x in (q, k, v)), sm_scale=scale, causal=causal,
                                   kv_lengths=L, bias=bt, return_lse=True)
    torch.cuda.synchronize()
    got, lse = to_np(got), to_np(lse)
    err = max_abs(got, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= (F32_TOL if f32 else HALF_TOL)
    empty = np.isposinf(want_lse)                        # [B, Hq, Lq]
    np.testing.assert_array_equal(np.isposinf(lse), empty)
    assert not np.any(got.transpose(0, 2, 1, 3)[empty]), "rows without a valid key must be exactly 0"
    fin = ~empty
    assert max_abs(lse[fin], want_lse[fin]) <= (1e-5 if f32 else 1e-3)


BWD_CASES = _flash_cases(60, 7, 1.2e8)


@pytest.mark.parametrize("dt,b,lq,lk,hq,hkv,d,causal,lengths,bias_shape", BWD_CASES)
def test_backward_sweep(device, dt, b, lq, lk, hq, hkv, d, causal, lengths, bias_shape):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    bias_grad = bias_shape is not None and (b + lq) % 2 == 0
    print(f"bwd {dt} B={b} Lq={lq} Lk={lk} Hq={hq} Hkv={hkv} D={d} causal={causal} "
          f"lengths={lengths} bias={bias_shape} bias_grad={bias_grad}", flush=True)
    q, k, v, do, bias = _inputs(202, dt, b, lq, lk, hq, hkv, d, bias_shape)
    scale = 1.0 / math.sqrt(d)
    mask = _mask(causal, lengths)
    db = None if bias is None else oracle.DenseBias(bias)
    f32 = dt == "f32"
    cdt = np.float64 if f32 else np.float32
    o, lse = oracle.xla_attention(q, k, v, mask=mask, bias=db, sm_scale=scale, strategy="dense", dtype=dt,
                                  compute_dtype=cdt, return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, bias=db, sm_scale=scale, dtype=dt,
                              compute_dtype=cdt, return_dbias=bias_grad)
    t = _tdt(dt)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got = flash_attention_bwd(*(to_dev(x, device, t) for x in (q, k, v, o, do)),
                              torch.from_numpy(np.asarray(lse, np.float32)).to(device), sm_scale=scale,
                              causal=causal, kv_lengths=L, bias=bt, bias_grad=bias_grad)
    torch.cuda.synchronize()
    names = ("dq", "dk", "dv", "dbias")
    if bias_grad:
        # the oracle's dbias is per (batch, query head); the kernel's is summed to the bias's shape
        bb, bh = bias_shape
        full = np.asarray(want[3], np.float64)
        want = (*want[:3], full.sum(axis=0, keepdims=True) if bb == 1 else full)
        want = (*want[:3], want[3].sum(axis=1, keepdims=True) if bh == 1 else want[3])
    for name, g, w in zip(names, got, want):
        g = to_np(g).astype(np.float64)
        w = np.asarray(w, np.float64)
        err = np.abs(g - w)
        if f32:
            tol = 1e-5 * max(1.0, float(np.max(np.abs(w)))) if w.size else 0.0
            assert (err.max() if err.size else 0.0) <= tol, f"{name}: max err {err.max():.3e} > {tol:.3e}"
        else:
            bad = err > ATOL + RTOL * np.abs(w)
            assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} outside tolerance, max {err.max():.3e}"
    if lengths is not None:
        for bi, n in enumerate(lengths):
            n = max(n, 0)
            assert torch.count_nonzero(got[1][bi, n:]) == 0 and torch.count_nonzero(got[2][bi, n:]) == 0


def _decode_cases(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["f32", "bf16", "f16"]))
        d, dv = int(rng.choice([64, 128, 256])), int(rng.choice([64, 128, 256]))
        b = int(rng.integers(1, 6))
        hkv = int(rng.choice([1, 2, 4]))
        hq = hkv * int(rng.choice([1, 2, 4, 8, 16]))
        lq = int(rng.choice([1, 1, 2, 3, 5]))
        s = int(rng.integers(1, 3000))
        if b * hq * lq * s * max(d, dv) > 2e8:
            continue
        lengths = [int(x) for x in rng.integers(-1, s + 3, size=b)] if rng.random() < 0.7 else None
        chunk = int(rng.choice([0, 128, 256, 512]))
        stream = str(rng.choice(["0", "1"]))
        out.append((dt, b, lq, s, hq, hkv, d, dv, lengths, chunk, stream))
    return out


@pytest.mark.parametrize("dt,b,lq,s,hq,hkv,d,dv,lengths,chunk,stream", _decode_cases(64, 33))
def test_splitkv_decode_sweep(device, monkeypatch, dt, b, lq, s, hq, hkv, d, dv, lengths, chunk, stream):
    import torch
    from probjax_amd.hip_attention import splitkv_decode

    print(f"decode {dt} B={b} Lq={lq} S={s} Hq={hq} Hkv={hkv} D={d} Dv={dv} lengths={lengths} "
          f"chunk={chunk} stream={stream}", flush=True)
    monkeypatch.setenv("PJX_DECODE_STREAM", stream)
    q, k, v = rng_normal(303, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, dv))
    if dt != "f32":
        q, k, v = (oracle.round_to(x, dt) for x in (q, k, v))
    scale = 1.0 / math.sqrt(d)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    f32 = dt == "f32"
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="dense", dtype=dt,
                                          compute_dtype=np.float64 if f32 else np.float32, return_lse=True)
    t = _tdt(dt)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = splitkv_decode(*(to_dev(x, device, t) for x in (q, k, v)), sm_scale=scale, kv_lengths=L,
                              chunk=chunk, return_lse=True)
    torch.cuda.synchronize()
    got, lse = to_np(got), to_np(lse)
    err = max_abs(got, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= (F32_TOL if f32 else HALF_TOL)
    empty = np.isposinf(want_lse)
    np.testing.assert_array_equal(np.isposinf(lse), empty)
    assert not np.any(got.transpose(0, 2, 1, 3)[empty])
    assert max_abs(lse[~empty], want_lse[~empty]) <= (1e-5 if f32 else 1e-3)


def _latent_cases(n, seed, prefill):
    rng = np.random.default_rng(seed)
    shapes = ((576, 512), (576, 576), (512, 512), (256, 256), (128, 128), (64, 64))
    out = []
    while len(out) < n:
        dt = str(rng.choice(["bf16", "f16"]))
        r, dv = shapes[int(rng.integers(len(shapes)))]
        b = int(rng.integers(1, 4))
        h = int(rng.integers(1, 41)) if not prefill else int(rng.integers(1, 5))
        lq = int(rng.choice([1, 1, 2, 3])) if not prefill else int(rng.integers(2, 300))
        s = int(rng.integers(1, 2500)) if not prefill else int(rng.integers(1, 400))
        if b * h * lq * s * r > 2e8:
            continue
        causal = prefill and bool(rng.random() < 0.5)
        lengths = [int(x) for x in rng.integers(-1, s + 3, size=b)] if rng.random() < 0.6 else None
        out.append((dt, b, lq, h, s, r, dv, causal, lengths))
    return out


def _latent_check(got, lse, want, want_lse):
    got, lse = to_np(got), to_np(lse)
    err = max_abs(got, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= HALF_TOL
    empty = np.isposinf(want_lse)
    np.testing.assert_array_equal(np.isposinf(lse), empty)
    assert not np.any(got.transpose(0, 2, 1, 3)[empty])
    assert max_abs(lse[~empty], want_lse[~empty]) <= 1e-3


@pytest.mark.parametrize("dt,b,lq,h,s,r,dv,causal,lengths", _latent_cases(32, 44, prefill=False))
def test_latent_decode_sweep(device, dt, b, lq, h, s, r, dv, causal, lengths):
    import torch
    from probjax_amd.hip_attention import mla_decode

    print(f"latent decode {dt} B={b} Lq={lq} H={h} S={s} R={r} Dv={dv} lengths={lengths}", flush=True)
    q, cache = (oracle.round_to(x, dt) for x in rng_normal(404, (b, lq, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, mask=mask, sm_scale=scale, strategy="dense",
                                          dtype=dt, return_lse=True)
    t = _tdt(dt)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = mla_decode(to_dev(q, device, t), to_dev(cache, device, t), sm_scale=scale, v_dim=dv,
                          kv_lengths=L, return_lse=True)
    torch.cuda.synchronize()
    _latent_check(got, lse, want[..., :dv], want_lse)


@pytest.mark.parametrize("dt,b,lq,h,s,r,dv,causal,lengths", _latent_cases(24, 55, prefill=True))
def test_latent_prefill_sweep(device, dt, b, lq, h, s, r, dv, causal, lengths):
    import torch
    from probjax_amd.hip_attention import mla_fwd

    print(f"latent prefill {dt} B={b} Lq={lq} H={h} S={s} R={r} Dv={dv} causal={causal} "
          f"lengths={lengths}", flush=True)
    q, cache = (oracle.round_to(x, dt) for x in rng_normal(505, (b, lq, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    mask = _mask(causal, lengths)
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, mask=mask, sm_scale=scale, strategy="dense",
                                          dtype=dt, return_lse=True)
    t = _tdt(dt)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = mla_fwd(to_dev(q, device, t), to_dev(cache, device, t), sm_scale=scale, v_dim=dv, causal=causal,
                       kv_lengths=L, return_lse=True)
    torch.cuda.synchronize()
    _latent_check(got, lse, want[..., :dv], want_lse)


def _latent_grad_cases(n, seed):
    rng = np.random.default_rng(seed)
    shapes = ((576, 512), (576, 576), (512, 512), (400, 400), (256, 256), (128, 128), (96, 96))
    out = []
    while len(out) < n:
        r, dv = shapes[int(rng.integers(len(shapes)))]
        dt = str(rng.choice(["bf16", "f16"] + (["f32"] if r <= 256 else [])))
        b, h = int(rng.integers(1, 3)), int(rng.integers(1, 5))
        lq, s = int(rng.integers(2, 260)), int(rng.integers(1, 330))
        if b * h * lq * s * r > 6e7:
            continue
        mask = [None, "causal", "kvlen", "window"][int(rng.integers(4))]
        bias = [None, None, "dense", "alibi"][int(rng.integers(4))]
        out.append((dt, b, lq, h, s, r, dv, mask, bias))
    return out


@pytest.mark.parametrize("dt,b,lq,h,s,r,dv,mask,bias", _latent_grad_cases(20, 66))
def test_latent_grad_sweep(device, dt, b, lq, h, s, r, dv, mask, bias):
    """Absorbed ``mla(q, cache, None, None)`` with gradients (dq, dcache) over
    random ranks (padded ones included), heads, lengths, masks and biases,
    checked as tests/test_gpu_mla_latent.py checks its cases."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M
    from tests.test_gpu_mla_latent import _check_grads, _mask_objects

    print(f"latent grads {dt} B={b} Lq={lq} H={h} S={s} R={r} Dv={dv} mask={mask} bias={bias}", flush=True)
    q, cache, do = rng_normal(606, (b, lq, h, r), (b, s, r), (b, lq, h, dv))
    low = dt != "f32"
    if low:
        q, cache, do = (oracle.round_to(x, dt) for x in (q, cache, do))
    scale = 1.0 / math.sqrt(192 if r == 576 else r)
    mm, om = _mask_objects(mask, b, lq, s, device)
    mb = ob = None
    if bias == "dense":
        (bt,) = rng_normal(607, (1, h, lq, s), scale=0.5)
        mb, ob = M.DenseBias(to_dev(bt, device, torch.float32)), oracle.DenseBias(bt)
    elif bias == "alibi":
        mb, ob = M.CausalAlibiBias(), oracle.CausalAlibiBias()
    t = _tdt(dt)
    tq, tc = (to_dev(x, device, t).requires_grad_(True) for x in (q, cache))
    out = A.mla(tq, tc, None, None, mask=mm, bias=mb, sm_scale=scale, v_dim=dv)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    shared = cache[:, :, None, :]
    cdt = np.float32 if low else np.float64
    want = oracle.xla_attention(q, shared, shared, mask=om, bias=ob, sm_scale=scale, strategy="dense",
                                dtype="f32", compute_dtype=cdt)
    err = max_abs(to_np(out), want[..., :dv])
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= (HALF_TOL if low else F32_TOL)
    dop = np.concatenate([do, np.zeros(do.shape[:-1] + (r - dv,), np.float32)], axis=-1)

    def grads(mode, compute):
        o, lse = oracle.xla_attention(q, shared, shared, mask=om, bias=ob, sm_scale=scale, strategy="dense",
                                      dtype=mode, compute_dtype=compute, return_lse=True)
        dq, dk, dv_ = attention_backward(q, shared, shared, o, dop, lse, mask=om, bias=ob, sm_scale=scale,
                                         dtype=mode, compute_dtype=compute)
        return np.asarray(dq, np.float64), (np.asarray(dk, np.float64) + np.asarray(dv_, np.float64))[:, :, 0]

    exact = grads("f32", np.float64)
    mode = grads(dt, np.float32) if low else (None, None)
    _check_grads([("dq", to_np(tq.grad), exact[0], mode[0]), ("dcache", to_np(tc.grad), exact[1], mode[1])], low)
