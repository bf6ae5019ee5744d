"""Parity at the BASELINE configurations' full sizes.

Prefill configs (2, 4) are checked against the oracle on sampled query rows
(causal row i is exactly attention of that row over keys 0..i, so a row
subset is an unmasked oracle call); decode configs (3, 5) are small enough for
the oracle in full.  Inputs are seeded numpy N(0,1) rounded to bf16 as the
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


def test_config2_full_size_sampled_rows(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import CausalMask

    B, L, H, D = 4, 4096, 16, 128
    q, k, v = _bf16_inputs(0, (B, L, H, D), (B, L, H, D), (B, L, H, D))
    out = to_np(flex_attention(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)), mask=CausalMask()))
    rng = np.random.default_rng(1)
    rows = np.unique(np.concatenate([[0, 1, 127, 128, 4095], rng.integers(0, L, 27)]))
    for b, h in [(0, 0), (3, 15), (2, 7)]:
        for i in rows:
            want = oracle.xla_attention(q[b : b + 1, i : i + 1, h : h + 1], k[b : b + 1, : i + 1, h : h + 1],
                                        v[b : b + 1, : i + 1, h : h + 1], sm_scale=1 / math.sqrt(D))
            assert max_abs(out[b, i, h], want[0, 0, 0]) <= BF16_TOL, (b, h, i)
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


def test_config4_full_size_sampled_rows(device):
    import torch
    from probjax_amd.attention import flex_attention
    from probjax_amd.masks import DenseBias, KVLenMask

    B, L, H, D = 2, 2048, 8, 64
    q, k, v = _bf16_inputs(3, (B, L, H, D), (B, L, H, D), (B, L, H, D))
    rng = np.random.default_rng(4)
    bias = (rng.standard_normal((H, L, L), dtype=np.float32) * np.float32(0.5))
    drop = int(round(0.1 * L)) + np.random.default_rng(0).integers(-16, 17, size=B)
    lengths = (L - drop).astype(np.int32)
    out = to_np(flex_attention(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)),
                               mask=KVLenMask(torch.from_numpy(lengths).to(device)),
                               bias=DenseBias(to_dev(bias[None], device, torch.float32))))
    rows = np.unique(np.concatenate([[0, L - 1], rng.integers(0, L, 14)]))
    for b in range(B):
        n = lengths[b]
        for h in (0, 5):
            for i in rows:
                want = oracle.xla_attention(q[b : b + 1, i : i + 1, h : h + 1], k[b : b + 1, :n, h : h + 1],
                                            v[b : b + 1, :n, h : h + 1],
                                            bias=oracle.DenseBias(bias[None, h : h + 1, i : i + 1, :n]),
                                            sm_scale=1 / 8)
                assert max_abs(out[b, i, h], want[0, 0, 0]) <= BF16_TOL, (b, h, i)


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
