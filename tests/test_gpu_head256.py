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
