"""Materialised latent attention (``mla`` with ``wk`` / ``wv``) on the GPU.

* ``pjx_mla_project`` (``K = C W_K^T``, ``V = C W_V^T`` per head, zero-padded
  to the head width) against numpy on the same bf16 / fp32 inputs: within one
  bf16 rounding step (the kernel and numpy sum in different orders, so a
  value near a rounding boundary may round the other way) and exactly zero in
  the padded channels; fp32 within 1e-5 relative.
* ``mla(q, cache, wk, wv)`` output and gradients in ``q, cache, wk, wv``
  against ``oracle.materialized_mla`` / ``materialized_mla_backward`` (the
  reference's ``_materialized_mla`` and its VJP): bf16 output max-abs <= 2e-2
  against the fp32 oracle from the same bf16-rounded inputs, gradients within
  probjax's gradient tolerance (atol 2e-2, rtol 1e-2, tests/test_attention.py:
  597-626) with atol scaled by max(1, max|ref| / 4) for gradients summed over
  many latent rows; fp32 output <= 1e-5 and gradients <= 1e-5 * max(1,
  max|ref|) against the float64 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,B,S,H,R,dk,dv,width", [
    ("bf16", 2, 200, 3, 72, 40, 24, 64),
    ("bf16", 1, 384, 4, 512, 128, 128, 128),
    ("bf16", 2, 33, 2, 12, 16, 12, 64),   # rank not a multiple of 8: element loads
    ("bf16", 2, 1900, 8, 72, 96, 64, 128),  # many tiles, ragged last row tile
    ("bf16", 1, 4096, 16, 512, 128, 128, 128),     # the bench's C5P shape
    ("bf16", 2, 2100, 12, 200, 100, 72, 128),      # ragged rows, padded head dims, rank 200
    ("f16", 3, 1500, 20, 136, 64, 64, 64),         # 1280 columns: 5 column tiles
    ("f32", 2, 200, 3, 72, 40, 24, 64),
    ("f32", 1, 130, 2, 20, 64, 128, 128),
])
def test_projection_matches_numpy(device, dtype, B, S, H, R, dk, dv, width):
    import torch
    from probjax_amd import hip_attention as hip

    print(f"project {dtype} B={B} S={S} H={H} R={R} dk={dk} dv={dv} width={width}", flush=True)
    cache, = rng_normal(60, (B, S, R))
    wk, wv = rng_normal(61, (H, dk, R), (H, dv, R), scale=1 / math.sqrt(R))
    from probjax_amd import native

    bf16 = dtype != "f32"   # 16-bit (bf16 or fp16)
    if bf16:
        cache, wk, wv = (oracle.round_to(x, dtype) for x in (cache, wk, wv))
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    k, v = hip.mla_project(*(to_dev(x, device, tdt) for x in (cache, wk, wv)), width=width)
    launched = native.last_launches()
    torch.cuda.synchronize()
    if bf16:
        ring = R % 8 == 0
        assert launched[0].startswith("mla_project_bf16_kernel" if ring else "mla_project_bf16_ragged_kernel"), launched
    for got, w, dim in ((k, wk, dk), (v, wv, dv)):
        got = to_np(got).astype(np.float64)
        want = (cache.reshape(-1, R).astype(np.float64) @ w.reshape(-1, R).astype(np.float64).T).reshape(B, S, H, dim)
        assert got.shape == (B, S, H, width)
        assert not got[..., dim:].any(), "padded channels must be zero"
        err = np.abs(got[..., :dim] - want)
        if bf16:
            step = 2.0 ** -7 if dtype == "bf16" else 2.0 ** -10   # one 16-bit rounding step
            assert (err <= step * np.abs(want) + 1e-6).all(), f"max err {err.max():.3e}"
        else:
            assert (err <= 1e-5 * np.maximum(1.0, np.abs(want))).all(), f"max err {err.max():.3e}"


def _masks(name, B, S):
    import torch
    from probjax_amd import masks as M

    dev = torch.device("cuda", 0)
    if name == "none":
        return None, None, None, None
    if name == "causal":
        return M.CausalMask(), None, oracle.CausalMask(), None
    if name == "kvlen_dense":
        lens = np.array([S, S // 3][:B], np.int32)
        (bias,) = rng_normal(62, (1, 1, S, S), scale=0.5)
        return (M.KVLenMask(torch.from_numpy(lens).to(dev)), M.DenseBias(torch.from_numpy(bias).to(dev)),
                oracle.KVLenMask(lens), oracle.DenseBias(bias))
    if name == "window_alibi":
        return (M.LocalWindowMask(40, 8), M.CausalAlibiBias(),
                oracle.LocalWindowMask(40, 8), oracle.CausalAlibiBias())
    if name == "key_padding":
        kl = np.random.default_rng(63).integers(1, S + 1, size=S).astype(np.int32)
        return (M.KeyPaddingMask(torch.from_numpy(kl).to(dev)), None, oracle.KeyPaddingMask(kl), None)
    raise KeyError(name)


CASES = [
    # dtype, mask, B, Lq, S, H, R, dk, dv
    ("f32", "none", 2, 32, 32, 4, 8, 16, 12),          # the reference's test shape
    ("f32", "causal", 2, 32, 32, 4, 8, 16, 16),
    ("bf16", "causal", 2, 256, 256, 4, 256, 128, 128),
    ("bf16", "kvlen_dense", 2, 160, 160, 2, 96, 64, 48),
    ("bf16", "window_alibi", 1, 192, 192, 4, 64, 96, 128),
    ("bf16", "key_padding", 2, 128, 128, 2, 128, 64, 64),
    ("f32", "kvlen_dense", 2, 96, 96, 2, 48, 64, 40),
]


@pytest.mark.parametrize("dtype,mask_name,B,Lq,S,H,R,dk,dv", CASES)
def test_materialized_mla_forward_and_grads(device, dtype, mask_name, B, Lq, S, H, R, dk, dv):
    import torch
    from probjax_amd import attention as A

    print(f"mla-mat {dtype} {mask_name} B={B} Lq={Lq} S={S} H={H} R={R} dk={dk} dv={dv}", flush=True)
    mask, bias, omask, obias = _masks(mask_name, B, S)
    q, cache, do = rng_normal(64, (B, Lq, H, dk), (B, S, R), (B, Lq, H, dv))
    wk, wv = rng_normal(65, (H, dk, R), (H, dv, R), scale=1 / math.sqrt(R))
    bf16 = dtype == "bf16"
    if bf16:
        q, cache, wk, wv, do = (oracle.round_bf16(x) for x in (q, cache, wk, wv, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    ts = [to_dev(x, device, tdt).requires_grad_(True) for x in (q, cache, wk, wv)]
    out = A.mla(*ts, mask=mask, bias=bias)
    assert out.shape == (B, Lq, H, dv)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    cdt = np.float32 if bf16 else np.float64
    kw = dict(mask=omask, bias=obias, dtype=dtype, compute_dtype=cdt)
    o_want = oracle.materialized_mla(q, cache, wk, wv, **kw)
    want = oracle.materialized_mla_backward(q, cache, wk, wv, do, **kw)
    got = [to_np(t.grad).astype(np.float64) for t in ts]
    names = ("dq", "dcache", "dwk", "dwv")
    if bf16:
        assert max_abs(to_np(out), o_want) <= 2e-2
        for nm, g, w in zip(names, got, want):
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(to_np(out), o_want) <= 1e-5
        for nm, g, w in zip(names, got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"
    # without autograd the same kernels run and give the same output
    with torch.no_grad():
        out2 = A.mla(*(t.detach() for t in ts), mask=mask, bias=bias)
    assert torch.equal(out.detach(), out2)


def test_projected_decode_routes(device, monkeypatch):
    """One query row per sequence over a long latent cache (a cached decode
    step): without gradients probjax's FLOP rule picks the absorbed form,
    which runs on the latent decode kernel; with gradients the call
    materialises.  Both against the oracle (xla_mla follows the same rule)."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H_
    from probjax_amd.masks import KVLenMask

    B, S, H, R, d = 2, 2048, 16, 512, 128
    print(f"mla projected decode B={B} S={S} H={H} R={R} d={d}", flush=True)
    lens = np.array([2048, 777], np.int32)
    q, cache = (oracle.round_bf16(x) for x in rng_normal(66, (B, 1, H, d), (B, S, R)))
    wk, wv = (oracle.round_bf16(x) for x in rng_normal(67, (H, d, R), (H, d, R), scale=1 / math.sqrt(R)))
    assert A._absorbed_cheaper(1, S, R, d, d)
    calls = []
    real = H_.mla_decode
    monkeypatch.setattr(H_, "mla_decode", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    ts = [to_dev(x, device, torch.bfloat16) for x in (q, cache, wk, wv)]
    mask = KVLenMask(torch.from_numpy(lens).to(device))
    got = A.mla(*ts, mask=mask)
    assert calls == [1], "the absorbed route runs the latent decode kernel"
    want = oracle.xla_mla(q, cache, wk, wv, mask=oracle.KVLenMask(lens), dtype="bf16")
    assert max_abs(to_np(got), want) <= 2e-2
    got_m = A.mla(ts[0].requires_grad_(True), *ts[1:], mask=mask)
    assert calls == [1], "with gradients the call materialises"
    want_m = oracle.materialized_mla(q, cache, wk, wv, mask=oracle.KVLenMask(lens), dtype="bf16")
    assert max_abs(to_np(got_m), want_m) <= 2e-2
