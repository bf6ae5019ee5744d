"""Parity at the BASELINE configurations' full sizes.

Every configuration is compared with the oracle over its whole output: all
(batch, head) slices and all query rows (the oracle runs config 2 in about
10 s of host time).  Inputs are seeded numpy N(0,1) rounded to bf16 as the
configurations specify.  Tolerance: bf16 max-abs <= 2e-2 vs the fp32 oracle.
"""

import math

import numpy as np
import pytest

import oracle
from tests._helpers import max_abs, to_dev, to_np

pytestmark = pytest.mark.gpu
BF16_TOL = 2e-2


def _bf16_inputs(seed, *shapes, scale=1.0):
    rng = np.random.default_rng(seed)
    return [oracle.round_bf16(rng.standard_normal(s, dtype=np.float32) * np.float32(scale)) for s in shapes]


def test_config2_full_size(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import CausalMask

    B, L, H, D = 4, 4096, 16, 128
    q, k, v = _bf16_inputs(0, (B, L, H, D), (B, L, H, D), (B, L, H, D))
    print(f"config 2 full size: B={B} L={L} H={H} D={D} causal", flush=True)
    out = to_np(flex_attention(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)), mask=CausalMask()))
    for b in range(B):
        want = oracle.xla_attention(q[b : b + 1], k[b : b + 1], v[b : b + 1], mask=oracle.CausalMask(),
                                    sm_scale=1 / math.sqrt(D))
        err = max_abs(out[b], want[0])
        print(f"  batch {b}: max-abs {err:.3e}", flush=True)
        assert err <= BF16_TOL, (b, err)
    # causal row 0 attends to key 0 only: output = v0 exactly (up to bf16 output rounding)
    np.testing.assert_array_equal(out[:, 0], v[:, 0])


def test_config3_full_size(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import KVLenMask

    B, S, Hq, Hkv, D = 32, 8192, 32, 8, 128
    lengths = np.random.default_rng(0).integers(512, 8193, size=B).astype(np.int32)
    q, k, v = _bf16_inputs(2, (B, 1, Hq, D), (B, S, Hkv, D), (B, S, Hkv, D))
    got = flex_attention(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)),
                         mask=KVLenMask(torch.from_numpy(lengths).to(device)), enable_gqa=True)
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=1 / math.sqrt(D))
    assert max_abs(to_np(got), want) <= BF16_TOL
    # keys past each length never matter: overwrite them and get the same bits
    k2, v2 = to_dev(k, device, torch.bfloat16), to_dev(v, device, torch.bfloat16)
    for b in range(B):
        k2[b, lengths[b]:] = 100.0
        v2[b, lengths[b]:] = -50.0
    got2 = flex_attention(to_dev(q, device, torch.bfloat16), k2, v2,
                          mask=KVLenMask(torch.from_numpy(lengths).to(device)), enable_gqa=True)
    assert torch.equal(got, got2)


def test_config4_full_size(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import DenseBias, KVLenMask

    B, L, H, D = 2, 2048, 8, 64
    q, k, v = _bf16_inputs(3, (B, L, H, D), (B, L, H, D), (B, L, H, D))
    rng = np.random.default_rng(4)
    bias = (rng.standard_normal((H, L, L), dtype=np.float32) * np.float32(0.5))
    drop = int(round(0.1 * L)) + np.random.default_rng(0).integers(-16, 17, size=B)
    lengths = (L - drop).astype(np.int32)
    print(f"config 4 full size: B={B} L={L} H={H} D={D} lengths={lengths.tolist()}", flush=True)
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    tb = to_dev(bias[None], device, torch.float32)
    tl = torch.from_numpy(lengths).to(device)
    got = flex_attention(tq, tk, tv, mask=KVLenMask(tl), bias=DenseBias(tb))
    out = to_np(got)
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), bias=oracle.DenseBias(bias[None]),
                                sm_scale=1 / 8)
    err = max_abs(out, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= BF16_TOL
    # keys past each length and their bias columns never matter
    k2, v2, b2 = tk.clone(), tv.clone(), tb.clone()
    for b in range(B):
        k2[b, lengths[b]:] = 100.0
        v2[b, lengths[b]:] = -50.0
    b2[..., int(lengths.max()):] = 1e4
    got2 = flex_attention(tq, k2, v2, mask=KVLenMask(tl), bias=DenseBias(b2))
    assert torch.equal(got, got2)


def test_config5_full_size(device):
    import torch
    from probjax_amd.attention import mla

    B, H, S, R = 16, 16, 4096, 576
    q, cache = _bf16_inputs(5, (B, 1, H, R), (B, S, R))
    scale = 1 / math.sqrt(192)
    got = mla(to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16), sm_scale=scale, v_dim=512)
    want = oracle.xla_mla(q, cache, sm_scale=scale)[..., :512]
    assert max_abs(to_np(got), want) <= BF16_TOL


def test_full_size_runs_are_deterministic(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import CausalMask

    g = torch.Generator(device=device)
    g.manual_seed(0)
    q, k, v = (torch.randn(4, 4096, 16, 128, generator=g, device=device).to(torch.bfloat16) for _ in range(3))
    a = flex_attention(q, k, v, mask=CausalMask())
    b = flex_attention(q, k, v, mask=CausalMask())
    assert torch.equal(a, b)
