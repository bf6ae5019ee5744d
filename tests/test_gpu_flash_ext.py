"""Extended masks and score modifiers on the GPU: forward output and LSE, and
dq / dk / dv through autograd, against the oracle (which restates probjax's
mask and bias classes).

Tolerances: bf16 output max-abs <= 2e-2 against the fp32 oracle from the
same bf16-rounded inputs, gradients within probjax's gradient tolerance
(atol 2e-2, rtol 1e-2, tests/test_attention.py:597-626) with atol scaled by
max(1, max|ref| / 4) for gradients larger than the usual ~4; fp32 output
max-abs <= 1e-5 and gradients <= 1e-5 * max(1, max|ref|) against the
float64 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _case(name, B, Lq, Lk):
    """(API mask, API bias, oracle mask, oracle bias) of a named case."""
    import torch
    from probjax_amd import masks as M

    dev = torch.device("cuda", 0)
    ids_np = np.stack([np.repeat(np.arange(4), -(-Lq // 4))[:Lq], np.repeat(np.arange(3), -(-Lq // 3))[:Lq]])
    ids_np = ids_np[:B].astype(np.int32)
    cases = {
        "bottom_right": (M.CausalFromBottomRightMask(Lq, Lk), None,
                         oracle.CausalFromBottomRightMask(Lq, Lk), None),
        "window": (M.LocalWindowMask(70, 20), None, oracle.LocalWindowMask(70, 20), None),
        "causal_window_kvlen": (
            M.CausalLocalWindowMask(100) & M.QKVLengthMask(Lq - 7, Lk - 30), None,
            oracle.CausalLocalWindowMask(100) & oracle.QKVLengthMask(Lq - 7, Lk - 30), None),
        "prefix": (M.PrefixLMMask(torch.tensor([50, 0][:B], device=dev)), None,
                   oracle.PrefixLMMask(np.array([50, 0][:B], np.int32)), None),
        "seqlen": (M.SeqLenMask(torch.tensor([200, 37][:B], device=dev)), None,
                   oracle.SeqLenMask(np.array([200, 37][:B], np.int32)), None),
        "segments": (M.SameSegmentMask(torch.from_numpy(ids_np).to(dev)), None,
                     oracle.SameSegmentMask(ids_np), None),
        "block_causal": (M.BlockDiagonalCausalMask(torch.from_numpy(ids_np).to(dev)), None,
                         oracle.BlockDiagonalCausalMask(ids_np), None),
        "alibi_causal": (M.CausalMask(), M.CausalAlibiBias(), oracle.CausalMask(), oracle.CausalAlibiBias()),
        "alibi_sym_const": (None, M.SymmetricAlibiBias() + M.ConstantBias(0.75), None,
                            oracle.SymmetricAlibiBias() + oracle.ConstantBias(0.75)),
        "decay_dense": (None, None, None, None),  # filled below (needs the dense tensor)
        "softcap": (M.CausalMask(), M.SoftCappingBias(2.0), oracle.CausalMask(), oracle.SoftCappingBias(2.0)),
        "headscale": (None, M.PerHeadScaleBias(torch.tensor([0.5, 2.0, 1.5, 3.0])), None,
                      oracle.PerHeadScaleBias(np.array([0.5, 2.0, 1.5, 3.0], np.float32))),
    }
    if name == "key_padding":
        # per-row counts, shorter than Lq: rows past the payload keep no key
        kl = np.random.default_rng(52).integers(0, Lk + 1, size=Lq - 20).astype(np.int32)
        return (M.KeyPaddingMask(torch.from_numpy(kl).to(dev)) & M.CausalMask(), None,
                oracle.KeyPaddingMask(kl) & oracle.CausalMask(), None)
    if name == "key_padding_2d":
        kl = np.random.default_rng(53).integers(0, Lk + 1, size=(B, Lq)).astype(np.int32)
        return (M.KeyPaddingMask(torch.from_numpy(kl).to(dev)), M.ConstantBias(0.5),
                oracle.KeyPaddingMask(kl), oracle.ConstantBias(0.5))
    if name == "decay_dense":
        (bias,) = rng_normal(50, (1, 4, Lq, Lk), scale=0.5)
        return (M.KVLenMask(torch.tensor([Lk, Lk // 2][:B], device=dev)),
                M.DistanceDecayBias(0.05) + M.DenseBias(torch.from_numpy(bias).to(dev)),
                oracle.KVLenMask(np.array([Lk, Lk // 2][:B], np.int32)),
                oracle.DistanceDecayBias(0.05) + oracle.DenseBias(bias))
    return cases[name]


CASES = [
    # name, B, Lq, Lk, Hq, Hkv, D
    ("bottom_right", 2, 100, 300, 4, 2, 128),
    ("window", 2, 384, 384, 4, 4, 64),
    ("causal_window_kvlen", 1, 512, 512, 4, 1, 128),
    ("prefix", 2, 256, 256, 4, 2, 64),
    ("seqlen", 2, 256, 256, 4, 4, 128),
    ("segments", 2, 300, 300, 4, 2, 128),
    ("block_causal", 2, 256, 256, 4, 4, 64),
    ("alibi_causal", 2, 320, 320, 4, 2, 128),
    ("alibi_sym_const", 2, 200, 200, 4, 4, 64),
    ("decay_dense", 2, 256, 256, 4, 2, 128),
    ("softcap", 2, 256, 256, 4, 4, 128),
    ("headscale", 2, 192, 192, 4, 1, 64),
    ("key_padding", 2, 256, 320, 4, 2, 128),
    ("key_padding_2d", 2, 160, 200, 4, 4, 64),
]


def _run(device, dtype, name, B, Lq, Lk, Hq, Hkv, D):
    import torch
    from probjax_amd import attention as A

    print(f"case {name} {dtype} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D}", flush=True)
    mask, bias, omask, obias = _case(name, B, Lq, Lk)
    q, k, v, do = rng_normal(51, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    scale = 1.0 / math.sqrt(D)
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.mha(tq, tk, tv, mask=mask, bias=bias, sm_scale=scale)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    cdt = np.float32 if bf16 else np.float64
    o_want, lse = oracle.xla_attention(q, k, v, mask=omask, bias=obias, sm_scale=scale, strategy="dense",
                                       dtype=dtype, compute_dtype=cdt, return_lse=True)
    want = attention_backward(q, k, v, o_want, do, lse, mask=omask, bias=obias, sm_scale=scale,
                              dtype=dtype, compute_dtype=cdt)
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv)]
    if bf16:
        assert max_abs(to_np(out), o_want) <= 2e-2
        for nm, g, w in zip(("dq", "dk", "dv"), got, want):
            # probjax's atol 2e-2 holds for gradients up to ~4 (the other cases);
            # a per-head scale of 3 sharpens the softmax and grows them to ~12, so
            # atol scales with the gradients' magnitude beyond 4 (the bf16 oracle
            # itself is 5e-2 from float64 there).
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(to_np(out), o_want) <= 1e-5
        for nm, g, w in zip(("dq", "dk", "dv"), got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"
    # the LSE of the modified, masked scores (natural log, +inf for empty rows)
    from probjax_amd.hip_attention import flash_attention_fwd

    e = A._eligible(tq.detach(), tk.detach(), tv.detach(), mask=mask, bias=bias, dropout_rate=0.0)
    plan = A._flash_plan(tq, tk, tv, e[0], e[1])
    _, glse = flash_attention_fwd(tq.detach(), tk.detach(), tv.detach(), sm_scale=scale,
                                  return_lse=True, **plan)
    glse = to_np(glse)
    np.testing.assert_array_equal(np.isposinf(glse), np.isposinf(lse))
    fin = np.isfinite(lse)
    assert max_abs(glse[fin], lse[fin]) <= (1e-3 if bf16 else 1e-5)


@pytest.mark.parametrize("name,B,Lq,Lk,Hq,Hkv,D", CASES)
def test_ext_bf16_forward_and_grads(device, name, B, Lq, Lk, Hq, Hkv, D):
    _run(device, "bf16", name, B, Lq, Lk, Hq, Hkv, D)


@pytest.mark.parametrize("name,B,Lq,Lk,Hq,Hkv,D", [c for c in CASES if c[0] in (
    "bottom_right", "causal_window_kvlen", "segments", "alibi_sym_const", "softcap", "headscale", "seqlen",
    "key_padding")])
def test_ext_f32_forward_and_grads(device, name, B, Lq, Lk, Hq, Hkv, D):
    _run(device, "f32", name, B, Lq, Lk, Hq, Hkv, D)
