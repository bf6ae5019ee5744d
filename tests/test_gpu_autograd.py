"""Gradients through the probjax-API mirror (torch autograd over the HIP
forward + backward) against the oracle's forward and backward.

probjax's own gradient tests compare implementations within atol 2e-2,
rtol 1e-2 (tests/test_attention.py:597-626); the same bar is used here for
bf16 against the fp32 oracle computed from the same bf16-rounded inputs.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want)
    assert (err <= ATOL + RTOL * np.abs(want)).all(), f"{what}: max err {err.max():.3e}"


def _leaves(device, *xs):
    import torch

    return [to_dev(x, device, torch.bfloat16).requires_grad_(True) for x in xs]


def _oracle_grads(q, k, v, do, *, mask, bias=None, scale):
    o, lse = oracle.xla_attention(q, k, v, mask=mask, bias=bias, sm_scale=scale, strategy="dense",
                                  dtype="bf16", return_lse=True)
    return o, attention_backward(q, k, v, o, do, lse, mask=mask, bias=bias, sm_scale=scale,
                                 dtype="bf16")


def test_flex_attention_causal_gqa_grad(device):
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    B, L, Hq, Hkv, D = 2, 384, 8, 2, 128
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(30, (B, L, Hq, D), (B, L, Hkv, D),
                                                           (B, L, Hkv, D), (B, L, Hq, D)))
    tq, tk, tv = _leaves(device, q, k, v)
    out = A.flex_attention(tq, tk, tv, mask=CausalMask(), enable_gqa=True)
    (out.float() * to_dev(do, device, out.dtype).float()).sum().backward()
    o_want, (dq, dk, dv) = _oracle_grads(q, k, v, do, mask=oracle.CausalMask(), scale=1 / math.sqrt(D))
    _close(to_np(out), o_want, "out")
    for name, t, w in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
        _close(to_np(t.grad), w, name)


def test_mha_kvlen_and_bias_grad_bias_gets_none(device):
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import DenseBias, KVLenMask

    B, L, H, D = 2, 256, 4, 64
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(31, (B, L, H, D), (B, L, H, D),
                                                           (B, L, H, D), (B, L, H, D)))
    bias = rng_normal(32, (1, H, L, L), scale=0.5)[0]
    lengths = np.array([256, 77], np.int32)
    tq, tk, tv = _leaves(device, q, k, v)
    tb = torch.from_numpy(bias).to(device).requires_grad_(True)
    out = A.mha(tq, tk, tv, mask=KVLenMask(torch.tensor(lengths, device=device)),
                bias=DenseBias(tb), sm_scale=0.125)
    (out.float() * to_dev(do, device, out.dtype).float()).sum().backward()
    mask, db = oracle.KVLenMask(lengths), oracle.DenseBias(bias)
    _, (dq, dk, dv) = _oracle_grads(q, k, v, do, mask=mask, bias=db, scale=0.125)
    for name, t, w in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
        _close(to_np(t.grad), w, name)
    # probjax's custom VJP gives the bias data no cotangent
    assert tb.grad is None
    assert torch.count_nonzero(tk.grad[1, 77:]) == 0


def test_decode_grad_uses_splitkv_primal(device, monkeypatch):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H
    from probjax_amd.masks import KVLenMask

    B, S, Hq, Hkv, D = 2, 2048, 8, 2, 128
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(33, (B, 1, Hq, D), (B, S, Hkv, D),
                                                           (B, S, Hkv, D), (B, 1, Hq, D)))
    lengths = np.array([2048, 1500], np.int32)
    calls = []
    real = H.splitkv_decode
    monkeypatch.setattr(H, "splitkv_decode", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    tq, tk, tv = _leaves(device, q, k, v)
    out = A.flex_attention(tq, tk, tv, mask=KVLenMask(torch.tensor(lengths, device=device)),
                           enable_gqa=True)
    assert calls, "the decode primal should be the split-KV kernel"
    (out.float() * to_dev(do, device, out.dtype).float()).sum().backward()
    _, (dq, dk, dv) = _oracle_grads(q, k, v, do, mask=oracle.KVLenMask(lengths), scale=1 / math.sqrt(D))
    for name, t, w in (("dq", tq, dq), ("dk", tk, dk), ("dv", tv, dv)):
        _close(to_np(t.grad), w, name)


def test_no_grad_inputs_take_the_plain_forward(device):
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    q, k, v = (to_dev(oracle.round_bf16(x), device, torch.bfloat16)
               for x in rng_normal(34, (1, 128, 2, 64), (1, 128, 2, 64), (1, 128, 2, 64)))
    out = A.flex_attention(q, k, v, mask=CausalMask())
    assert out.grad_fn is None
    tq = q.clone().requires_grad_(True)
    out2 = A.flex_attention(tq, k, v, mask=CausalMask())
    assert out2.grad_fn is not None
    assert torch.equal(out, out2.detach())


def test_config1_f32_grad(device):
    """Config 1 (fp32 causal 1x512x4x64) through flex_attention with gradients,
    against the float64 oracle: max-abs <= 1e-5 * max(1, max|ref|)."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    q, k, v, do = rng_normal(35, (1, 512, 4, 64), (1, 512, 4, 64), (1, 512, 4, 64), (1, 512, 4, 64))
    tq, tk, tv = (to_dev(x, device, torch.float32).requires_grad_(True) for x in (q, k, v))
    out = A.flex_attention(tq, tk, tv, mask=CausalMask())
    (out * to_dev(do, device, torch.float32)).sum().backward()
    o, lse = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / 8, strategy="dense",
                                  compute_dtype=np.float64, return_lse=True)
    assert float(np.max(np.abs(to_np(out) - o))) <= 1e-5
    want = attention_backward(q, k, v, o, do, lse, mask=oracle.CausalMask(), sm_scale=1 / 8,
                              compute_dtype=np.float64)
    for name, t, w in (("dq", tq, want[0]), ("dk", tk, want[1]), ("dv", tv, want[2])):
        err = float(np.max(np.abs(to_np(t.grad).astype(np.float64) - w)))
        assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{name}: {err:.3e}"
