"""Absorbed latent attention beyond decode: ``mla(q, cache, None, None, ...)``
with any query length, masks, biases and gradients on the GPU.

probjax's absorbed ``mla`` (kernels/latent_attention.py:79-197, 636-766) is
attention over K = V = the shared latent; its custom VJP (:752-766)
differentiates ``mha`` over the latent broadcast to every head, so
``dcache = sum_heads (dK + dV)``.  The oracle here is ``oracle.xla_mla``
(the reference's CPU path, :591-625) for the output and
``oracle.backward.attention_backward`` with the latent as the one shared KV
head for ``(dq, dK, dV)``; ``dcache = dK + dV``.  A call returning only the
first ``v_dim`` columns has zero gradient in the others, so the oracle's
output gradient is zero-padded to the latent width.

Folded calls (``[B, Q*H, 1, R]``, layers/latent_attention.py:458-469, 633-684)
are the same attention with one query head.

Tolerances: bf16 output max-abs <= 2e-2 against the fp32 oracle from the same
bf16-rounded inputs (its output is not rounded to bf16 again: two independent
bf16 roundings of an output in [4, 8) can land one ulp, 3.1e-2, apart).  bf16 gradients are
checked against the exact (float64, no bf16 rounding of P and dS) gradient
of those inputs: within probjax's gradient tolerance (atol 2e-2, rtol 1e-2,
tests/test_attention.py:597-626) with atol scaled by max(1, max|ref| / 4),
since these gradients sum over hundreds of keys or every head and query row,
and with an RMS error at most 1.5x that of the oracle's own bf16-mode
gradient (which rounds P and dS as the reference does).  Against the bf16-mode
oracle directly, two independent sets of bf16 roundings add up: on the
causal + bias case at L = 1024 the kernel is 2.9e-2 (max) / 7.6e-4 (RMS) from
float64 for dq, the bf16-mode oracle 3.2e-2 / 7.8e-4, and the two 4.7e-2
apart.  fp32 (latent width <= 128) output <= 1e-5 and gradients
<= 1e-5 * max(1, max|ref|) against the float64 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _mask_objects(kind, B, Lq, Lk, device):
    """(mirror mask, oracle mask) of one case."""
    import torch
    from probjax_amd import masks as M

    if kind is None:
        return None, None
    if kind == "causal":
        return M.CausalMask(), oracle.CausalMask()
    if kind == "kvlen":
        L = np.array([Lk, max(1, Lk // 3)] + [Lk - 7] * (B - 2), np.int32)[:B]
        return M.KVLenMask(torch.from_numpy(L).to(device)), oracle.KVLenMask(L)
    if kind == "kvlen_empty":
        L = np.array([0] + [Lk - 5] * (B - 1), np.int32)
        return M.KVLenMask(torch.from_numpy(L).to(device)), oracle.KVLenMask(L)
    if kind == "window":
        return M.CausalLocalWindowMask(96), oracle.CausalLocalWindowMask(96)
    raise AssertionError(kind)


def _check_grads(pairs, bf16):
    """pairs: (name, kernel gradient, exact float64 gradient, bf16-mode oracle
    gradient or None)."""
    for nm, g, w, wb in pairs:
        g = np.asarray(g, np.float64)
        w = np.asarray(w, np.float64)
        if bf16:
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e} (atol {atol:.3e})"
            rms = float(np.sqrt(np.mean(err ** 2)))
            rms_ref = float(np.sqrt(np.mean((np.asarray(wb, np.float64) - w) ** 2)))
            print(f"  {nm}: max err {err.max():.3e}, rms {rms:.3e} (bf16 oracle rms {rms_ref:.3e})", flush=True)
            assert rms <= 1.5 * rms_ref + 1e-7, f"{nm}: rms {rms:.3e} against the bf16 oracle's {rms_ref:.3e}"
        else:
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"


# (name, dtype, B, Lq, Lk, H, R, v_dim, mask, bias, folded, grad)
_CASES = [
    ("causal_r576_full", "bf16", 2, 1024, 1024, 16, 576, 576, "causal", None, False, True),
    ("causal_bias_r576_v512", "bf16", 2, 1024, 1024, 16, 576, 512, "causal", "dense", False, True),
    ("folded_kvlen_bias", "bf16", 2, 64, 640, 16, 576, 512, "kvlen", "dense_folded", True, True),
    ("folded_causal", "bf16", 1, 40, 300, 8, 576, 576, "causal", None, True, False),
    ("causal_r512", "bf16", 2, 512, 512, 8, 512, 512, "causal", None, False, True),
    ("window_alibi_r576", "bf16", 2, 200, 200, 4, 576, 512, "window", "alibi", False, True),
    ("kvlen_empty_r576", "bf16", 3, 96, 333, 4, 576, 576, "kvlen_empty", None, False, True),
    ("ragged_r400", "bf16", 1, 130, 170, 4, 400, 400, None, "dense", False, True),
    ("causal_r128_bf16", "bf16", 2, 256, 256, 4, 128, 128, "causal", "dense", False, True),
    ("causal_r128_f32", "f32", 2, 160, 160, 4, 128, 128, "causal", None, False, True),
    ("kvlen_r96_f32", "f32", 2, 64, 200, 2, 96, 96, "kvlen", None, False, True),
    # the bench shape's widths without bias: 16 head groups of fp32 partials
    ("causal_r576_v512", "bf16", 1, 640, 700, 16, 576, 512, "causal", None, False, True),
    # one head: a single group writes dcache directly (no partials)
    ("one_head_kvlen_r576", "bf16", 2, 200, 300, 1, 576, 512, "kvlen", None, False, True),
]


@pytest.mark.parametrize("case", _CASES, ids=[c[0] for c in _CASES])
def test_absorbed_mla_forward_and_grads(device, case):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    name, dtype, B, Lq, Lk, H, R, v_dim, mkind, bkind, folded, grad = case
    bf16 = dtype == "bf16"
    print(f"latent {name}: {dtype} B={B} Lq={Lq} Lk={Lk} H={H} R={R} v_dim={v_dim} mask={mkind} "
          f"bias={bkind} folded={folded} grad={grad}", flush=True)
    seed = 300 + _CASES.index(case)
    q, cache = rng_normal(seed, (B, Lq, H, R), (B, Lk, R))
    (do,) = rng_normal(seed + 1, (B, Lq, H, v_dim))
    if bf16:
        q, cache, do = (oracle.round_bf16(x) for x in (q, cache, do))
    scale = 1.0 / math.sqrt(192 if R == 576 else R)
    if folded:
        q = q.reshape(B, Lq * H, 1, R)
        do = do.reshape(B, Lq * H, 1, v_dim)
    qb, hb = q.shape[1], q.shape[2]
    mm, om = _mask_objects(mkind, B, qb, Lk, device)
    mb = ob = None
    bias = None
    if bkind == "dense":
        (bias,) = rng_normal(seed + 2, (1, hb, qb, Lk), scale=0.5)
    elif bkind == "dense_folded":
        (bias,) = rng_normal(seed + 2, (B, 1, qb, Lk), scale=0.5)
    if bias is not None:
        mb, ob = M.DenseBias(to_dev(bias, device, torch.float32)), oracle.DenseBias(bias)
    elif bkind == "alibi":
        mb, ob = M.CausalAlibiBias(), oracle.CausalAlibiBias()

    tdt = torch.bfloat16 if bf16 else torch.float32
    tq = to_dev(q, device, tdt).requires_grad_(grad)
    tc = to_dev(cache, device, tdt).requires_grad_(grad)
    out = A.mla(tq, tc, None, None, mask=mm, bias=mb, sm_scale=scale, v_dim=v_dim)
    assert out.shape == q.shape[:3] + (v_dim,)
    if grad:
        (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    cdt = np.float32 if bf16 else np.float64
    shared = cache[:, :, None, :]
    # the fp32 oracle on the same (16-bit-rounded) inputs: its output is not
    # rounded again, so a bf16 output is held to the bar of the other bf16 tests
    want, lse = oracle.xla_attention(q, shared, shared, mask=om, bias=ob, sm_scale=scale, strategy="dense",
                                     dtype="f32", compute_dtype=cdt, return_lse=True)
    err = max_abs(to_np(out), want[..., :v_dim])
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= (2e-2 if bf16 else 1e-5)
    if not grad:
        return
    dop = np.concatenate([do, np.zeros(do.shape[:-1] + (R - v_dim,), np.float32)], axis=-1)

    def grads(dt, compute):
        o, lse_ = oracle.xla_attention(q, shared, shared, mask=om, bias=ob, sm_scale=scale, strategy="dense",
                                       dtype=dt, compute_dtype=compute, return_lse=True)
        dq_, dk_, dv_ = attention_backward(q, shared, shared, o, dop, lse_, mask=om, bias=ob, sm_scale=scale,
                                           dtype=dt, compute_dtype=compute)
        return np.asarray(dq_, np.float64), (np.asarray(dk_, np.float64) + np.asarray(dv_, np.float64))[:, :, 0]

    exact = grads("f32", np.float64)
    mode = grads("bf16", np.float32) if bf16 else (None, None)
    _check_grads([("dq", to_np(tq.grad), exact[0], mode[0]), ("dcache", to_np(tc.grad), exact[1], mode[1])], bf16)


def test_absorbed_prefill_routes(device, monkeypatch):
    """Decode-shaped calls without gradients (up to 128 folded rows: each 16
    form a row group of the split-KV latent kernel) keep that kernel; a causal
    mask, a bias, Lq*H > 128 or a gradient take the latent flash kernels (one
    call each, through pjx_mla_fwd / pjx_mla_bwd)."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as hip
    from probjax_amd import masks as M

    calls = []
    for nm in ("mla_decode", "mla_fwd", "mla_bwd"):
        orig = getattr(hip, nm)

        def wrap(*a, _o=orig, _n=nm, **k):
            calls.append(_n)
            return _o(*a, **k)

        monkeypatch.setattr(hip, nm, wrap)
    q, c = rng_normal(40, (2, 1, 16, 576), (2, 300, 576))
    tq, tc = to_dev(q, device, torch.bfloat16), to_dev(c, device, torch.bfloat16)
    A.mla(tq, tc, sm_scale=0.1, v_dim=512)
    assert calls == ["mla_decode"]
    calls.clear()
    A.mla(tq, tc, sm_scale=0.1, mask=M.CausalMask())
    assert calls == ["mla_fwd"]
    calls.clear()
    q2 = to_dev(rng_normal(41, (2, 4, 16, 576))[0], device, torch.bfloat16)
    A.mla(q2, tc, sm_scale=0.1)  # 64 folded rows: four row groups of the decode
    assert calls == ["mla_decode"]
    calls.clear()
    q3 = to_dev(rng_normal(42, (2, 9, 16, 576))[0], device, torch.bfloat16)
    A.mla(q3, tc, sm_scale=0.1)  # 144 folded rows: a query block for the flash kernels
    assert calls == ["mla_fwd"]
    calls.clear()
    tq.requires_grad_(True)
    A.mla(tq, tc, sm_scale=0.1).float().sum().backward()
    assert calls == ["mla_fwd", "mla_bwd"]


def test_absorbed_prefill_deterministic(device):
    """Two runs give bitwise-identical outputs and gradients (the cache
    gradient's head-group partials are summed in a fixed order)."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    q, c, do = rng_normal(42, (1, 384, 16, 576), (1, 384, 576), (1, 384, 16, 512))
    res = []
    for _ in range(2):
        tq = to_dev(q, device, torch.bfloat16).requires_grad_(True)
        tc = to_dev(c, device, torch.bfloat16).requires_grad_(True)
        out = A.mla(tq, tc, mask=M.CausalMask(), sm_scale=1 / math.sqrt(192), v_dim=512)
        (out.float() * to_dev(do, device, torch.float32)).sum().backward()
        res.append((out.detach(), tq.grad, tc.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)
