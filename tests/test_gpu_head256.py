"""Head dims above 128 on the GPU (bf16): D = 256 natively, D = 160 / 192 /
200 zero-padded to 256 (the reference's fused route takes D <= 256,
layers/attention.py:1193-1195, padding blocks to next_power_of_2(head_dim),
kernels/attention.py:2168).  Forward and backward (dq, dk, dv, and the dense
bias gradient through ``dot_product_attention``) against the oracle, with
causal, KV-length, dense-bias, GQA and extended (window + ALiBi) cases.

Tolerances: output max-abs <= 2e-2 against the fp32 oracle from the same
bf16-rounded inputs; gradients within probjax's gradient tolerance (atol 2e-2
scaled by max(1, max|ref| / 4), rtol 1e-2).
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

# (name, B, Lq, Lk, Hq, Hkv, D, mask, bias)
CASES = [
    ("causal_d256", 2, 384, 384, 4, 4, 256, "causal", None),
    ("gqa_nomask_d256", 1, 200, 333, 8, 2, 256, None, None),
    ("kvlen_bias_d256", 2, 160, 256, 2, 1, 256, "kvlen", "dense"),
    ("window_alibi_d256", 1, 300, 300, 2, 2, 256, "window", "alibi"),
    ("causal_d192", 2, 256, 256, 2, 2, 192, "causal", None),
    ("kvlen_d160", 2, 100, 180, 4, 2, 160, "kvlen", None),
    ("bias_d200", 1, 128, 128, 2, 2, 200, None, "dense"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_wide_head_forward_and_grads(device, case):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    name, B, Lq, Lk, Hq, Hkv, D, mkind, bkind = case
    print(f"wide head {name}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} mask={mkind} bias={bkind}",
          flush=True)
    seed = 400 + CASES.index(case)
    q, k, v, do = rng_normal(seed, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    lens = np.array([Lk, Lk // 3][:B], np.int32)
    mask, omask = {
        None: (None, None),
        "causal": (M.CausalMask(), oracle.CausalMask()),
        "kvlen": (M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)),
        "window": (M.LocalWindowMask(64, 32), oracle.LocalWindowMask(64, 32)),
    }[mkind]
    bias = ob = mb = None
    tb = None
    if bkind == "dense":
        (bias,) = rng_normal(seed + 1, (B, Hq, Lq, Lk), scale=0.5)
        tb = to_dev(bias, device, torch.float32).requires_grad_(True)
        mb, ob = M.DenseBias(tb), oracle.DenseBias(bias)
    elif bkind == "alibi":
        mb, ob = M.SymmetricAlibiBias(), oracle.SymmetricAlibiBias()
    tq, tk, tv = (to_dev(x, device, torch.bfloat16).requires_grad_(True) for x in (q, k, v))
    out = A.dot_product_attention(tq, tk, tv, mask=mask, bias=mb)
    assert out.shape == (B, Lq, Hq, D)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    scale = 1.0 / math.sqrt(D)
    o, lse = oracle.xla_attention(q, k, v, mask=omask, bias=ob, sm_scale=scale, strategy="dense", dtype="bf16",
                                  return_lse=True)
    res = attention_backward(q, k, v, o, do, lse, mask=omask, bias=ob, sm_scale=scale, dtype="bf16",
                             return_dbias=tb is not None)
    err = max_abs(to_np(out), o)
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= 2e-2
    pairs = [("dq", tq, res[0]), ("dk", tk, res[1]), ("dv", tv, res[2])]
    if tb is not None:
        pairs.append(("dbias", tb, res[3]))
    for nm, t, w in pairs:
        g = to_np(t.grad).astype(np.float64)
        w = np.asarray(w, np.float64)
        atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
        e = np.abs(g - w)
        assert (e <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {e.max():.3e}"


def test_d256_masked_keys_do_not_matter(device):
    """Keys past each KV length are never read: overwriting them leaves the
    forward output and the query gradient bitwise unchanged, and their key /
    value gradients are exactly zero."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    B, L, H, D = 2, 256, 2, 256
    q, k, v, do = rng_normal(450, (B, L, H, D), (B, L, H, D), (B, L, H, D), (B, L, H, D))
    lens = torch.tensor([200, 77], dtype=torch.int32, device=device)
    res = []
    for poison in (False, True):
        tk, tv = to_dev(k, device, torch.bfloat16), to_dev(v, device, torch.bfloat16)
        if poison:
            for b in range(B):
                tk[b, int(lens[b]):] = 100.0
                tv[b, int(lens[b]):] = -50.0
        tq = to_dev(q, device, torch.bfloat16).requires_grad_(True)
        tk.requires_grad_(True)
        tv.requires_grad_(True)
        out = A.flex_attention(tq, tk, tv, mask=M.KVLenMask(lens))
        (out.float() * to_dev(do, device, torch.float32)).sum().backward()
        res.append((out.detach(), tq.grad, tk.grad, tv.grad))
    assert torch.equal(res[0][0], res[1][0]) and torch.equal(res[0][1], res[1][1])
    for b in range(B):
        n = int(lens[b])
        assert not res[1][2][b, n:].any() and not res[1][3][b, n:].any()


# fp32 at head dims above 128: (name, B, Lq, Lk, Hq, Hkv, D, mask, bias)
F32_CASES = [
    ("f32_causal_d256", 2, 200, 200, 4, 2, 256, "causal", None),
    ("f32_kvlen_bias_d256", 2, 130, 170, 2, 1, 256, "kvlen", "dense"),
    ("f32_window_alibi_d256", 1, 150, 150, 2, 2, 256, "window", "alibi"),
    ("f32_segments_d256", 2, 96, 96, 2, 2, 256, "segments", None),
    ("f32_softcap_d192", 1, 120, 140, 4, 4, 192, "causal", "softcap"),
    ("f32_nomask_d160", 2, 64, 100, 4, 1, 160, None, None),
]


@pytest.mark.parametrize("case", F32_CASES, ids=[c[0] for c in F32_CASES])
def test_f32_wide_head_forward_and_grads(device, case):
    """fp32 at D = 256 (and 160 / 192 zero-padded to it) on the fp32 wide
    kernels (v_mfma_f32_16x16x4f32): output and LSE within 1e-5 of the
    float64 oracle, dq / dk / dv (and dbias) within 1e-5 * max(1, max|ref|),
    with causal, KV-length, window, segment-id masks, a dense bias, ALiBi and
    soft capping; the launched instances are asserted."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M
    from probjax_amd import native
    from probjax_amd.hip_attention import flash_attention_fwd

    name, B, Lq, Lk, Hq, Hkv, D, mkind, bkind = case
    print(f"fp32 wide head {name}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} mask={mkind} bias={bkind}",
          flush=True)
    seed = 460 + F32_CASES.index(case)
    q, k, v, do = rng_normal(seed, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    lens = np.array([Lk, Lk // 3][:B], np.int32)
    ids = np.stack([np.repeat(np.arange(3), -(-Lq // 3))[:Lq], np.repeat(np.arange(5), -(-Lq // 5))[:Lq]])[:B]
    ids = ids.astype(np.int32)
    mask, omask = {
        None: (None, None),
        "causal": (M.CausalMask(), oracle.CausalMask()),
        "kvlen": (M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)),
        "window": (M.LocalWindowMask(40, 10), oracle.LocalWindowMask(40, 10)),
        "segments": (M.SameSegmentMask(torch.from_numpy(ids).to(device)), oracle.SameSegmentMask(ids)),
    }[mkind]
    ob = mb = tb = None
    if bkind == "dense":
        (bias,) = rng_normal(seed + 1, (B, Hq, Lq, Lk), scale=0.5)
        tb = to_dev(bias, device, torch.float32).requires_grad_(True)
        mb, ob = M.DenseBias(tb), oracle.DenseBias(bias)
    elif bkind == "alibi":
        mb, ob = M.CausalAlibiBias(), oracle.CausalAlibiBias()
    elif bkind == "softcap":
        mb, ob = M.SoftCappingBias(2.0), oracle.SoftCappingBias(2.0)
    tq, tk, tv = (to_dev(x, device, torch.float32).requires_grad_(True) for x in (q, k, v))
    out = A.dot_product_attention(tq, tk, tv, mask=mask, bias=mb)
    (out * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    scale = 1.0 / math.sqrt(D)
    o, lse = oracle.xla_attention(q, k, v, mask=omask, bias=ob, sm_scale=scale, strategy="dense",
                                  compute_dtype=np.float64, return_lse=True)
    res = attention_backward(q, k, v, o, do, lse, mask=omask, bias=ob, sm_scale=scale, compute_dtype=np.float64,
                             return_dbias=tb is not None)
    err = max_abs(to_np(out), o)
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= 1e-5
    pairs = [("dq", tq, res[0]), ("dk", tk, res[1]), ("dv", tv, res[2])]
    if tb is not None:
        pairs.append(("dbias", tb, res[3]))
    for nm, t, w in pairs:
        g = to_np(t.grad).astype(np.float64)
        e = float(np.max(np.abs(g - np.asarray(w, np.float64))))
        print(f"  {nm} max-abs {e:.3e}", flush=True)
        assert e <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), nm
    # the forward instance and its LSE (+inf exactly for rows with no key)
    e = A._eligible(tq.detach(), tk.detach(), tv.detach(), mask=mask, bias=mb, dropout_rate=0.0)
    pq, pk, pv = (A._pad_features(t.detach(), 256) for t in (tq, tk, tv))
    plan = A._flash_plan(pq, pk, pv, e[0], e[1])
    _, glse = flash_attention_fwd(pq, pk, pv, sm_scale=scale, return_lse=True, **plan)
    launched = native.last_launches()
    torch.cuda.synchronize()
    hb = "true" if plan.get("bias") is not None else "false"
    mods = "true" if plan.get("mods") is not None else "false"
    assert launched == [f"flash_fwd_f32_wide_kernel<256, {hb}, {mods}>"], launched
    glse = to_np(glse)
    np.testing.assert_array_equal(np.isposinf(glse), np.isposinf(lse))
    fin = np.isfinite(lse)
    assert max_abs(glse[fin], lse[fin]) <= 1e-5
