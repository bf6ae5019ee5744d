"""Head dims the kernels do not carry natively (any D <= 128 other than 64 and
128) on the GPU: the route zero-pads Q, K and V to 64 or 128 features and
slices the output and the gradients back, as the reference pads its blocks to
next_power_of_2(head_dim) (kernels/attention.py:2168).  Forward, backward and
the split-KV decode, against the oracle at the true head dim.

Tolerances: bf16 output max-abs <= 2e-2 against the fp32 oracle from the same
bf16-rounded inputs, gradients within probjax's gradient tolerance (atol
2e-2 scaled by max(1, max|ref| / 4), rtol 1e-2); fp32 output <= 1e-5 and
gradients <= 1e-5 * max(1, max|ref|) against the float64 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

CASES = [
    # dtype, B, L, Hq, Hkv, D, mask
    ("bf16", 2, 200, 4, 2, 96, "causal"),
    ("bf16", 1, 256, 2, 2, 32, "none"),
    ("f32", 2, 130, 2, 1, 80, "kvlen"),
    ("f32", 1, 96, 2, 2, 8, "causal"),
]


@pytest.mark.parametrize("dtype,B,L,Hq,Hkv,D,mask_name", CASES)
def test_padded_head_dim_forward_and_grads(device, dtype, B, L, Hq, Hkv, D, mask_name):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    print(f"head dim {D} {dtype} B={B} L={L} Hq={Hq} Hkv={Hkv} {mask_name}", flush=True)
    q, k, v, do = rng_normal(100 + D, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, L, Hq, D))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v, do = (oracle.round_bf16(x) for x in (q, k, v, do))
    tdt = torch.bfloat16 if bf16 else torch.float32
    lens = np.array([L, L // 3][:B], np.int32)
    mask, omask = {
        "none": (None, None),
        "causal": (M.CausalMask(), oracle.CausalMask()),
        "kvlen": (M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)),
    }[mask_name]
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.flex_attention(tq, tk, tv, mask=mask, enable_gqa=Hq != Hkv)
    assert out.shape == (B, L, Hq, D)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    scale = 1.0 / math.sqrt(D)
    cdt = np.float32 if bf16 else np.float64
    o, lse = oracle.xla_attention(q, k, v, mask=omask, sm_scale=scale, strategy="dense", dtype=dtype,
                                  compute_dtype=cdt, return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=omask, sm_scale=scale, dtype=dtype, compute_dtype=cdt)
    got = [to_np(t.grad).astype(np.float64) for t in (tq, tk, tv)]
    for t, shape in zip((tq, tk, tv), (q.shape, k.shape, v.shape)):
        assert tuple(t.grad.shape) == shape
    if bf16:
        assert max_abs(to_np(out), o) <= 2e-2
        for nm, g, w in zip(("dq", "dk", "dv"), got, want):
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            err = np.abs(g - w)
            assert (err <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {err.max():.3e}"
    else:
        assert max_abs(to_np(out), o) <= 1e-5
        for nm, g, w in zip(("dq", "dk", "dv"), got, want):
            err = float(np.max(np.abs(g - w)))
            assert err <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {err:.3e}"


def test_padded_head_dim_equals_explicit_padding(device):
    """The padded route gives bit-for-bit what the 128-wide kernel gives on
    explicitly zero-padded inputs."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    q, k, v = rng_normal(110, (1, 300, 2, 72), (1, 300, 2, 72), (1, 300, 2, 72))
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    got = A.mha(tq, tk, tv, mask=CausalMask(), sm_scale=0.1)
    pad = [torch.nn.functional.pad(x, (0, 56)) for x in (tq, tk, tv)]
    want = A.mha(*pad, mask=CausalMask(), sm_scale=0.1)[..., :72]
    assert torch.equal(got, want)


@pytest.mark.parametrize("D", [40, 96])
def test_padded_head_dim_splitkv_decode(device, D):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H
    from probjax_amd.masks import KVLenMask

    print(f"split-KV decode head dim {D}", flush=True)
    lengths = np.array([1500, 333], np.int32)
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(111, (2, 1, 8, D), (2, 1536, 2, D), (2, 1536, 2, D)))
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    tl = torch.from_numpy(lengths).to(device)
    assert A.use_splitkv(tq, tk, mask=KVLenMask(tl))
    calls = []
    real = H.splitkv_decode
    H.splitkv_decode = lambda *a, **kw: calls.append(1) or real(*a, **kw)
    try:
        got = A.mha(tq, tk, tv, mask=KVLenMask(tl), sm_scale=1 / math.sqrt(D))
    finally:
        H.splitkv_decode = real
    assert calls, "the padded decode did not run the split-KV kernel"
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=1 / math.sqrt(D))
    assert got.shape == (2, 1, 8, D)
    assert max_abs(to_np(got), want) <= 2e-2
    o2, lse2 = A.splitkv_forward(tq, tk, tv, sm_scale=1 / math.sqrt(D), kv_lengths=tl, return_lse=True)
    assert o2.shape == (2, 1, 8, D) and lse2.shape == (2, 8, 1)
    assert max_abs(to_np(o2), want) <= 2e-2
