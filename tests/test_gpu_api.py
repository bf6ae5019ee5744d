"""The probjax-API mirror on the GPU: each BASELINE configuration's call,
expressed as probjax expresses it, against the CPU oracle (reduced sizes where
the oracle would be slow; full-size properties in tests/test_gpu_fullsize.py).

Tolerances: fp32 max-abs <= 1e-5; bf16 max-abs <= 2e-2 against an fp32 oracle
computed from the same bf16-rounded inputs.
"""

import math

import numpy as np
import pytest

import oracle
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _bf(x, device):
    import torch

    return to_dev(oracle.round_bf16(x), device, torch.bfloat16)


def test_config1_flex_attention_causal_f32(device):
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    q, k, v = rng_normal(0, (1, 512, 4, 64), (1, 512, 4, 64), (1, 512, 4, 64))
    want = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / 8)
    got = A.flex_attention(*(to_dev(x, device, torch.float32) for x in (q, k, v)), mask=CausalMask())
    assert max_abs(to_np(got), want) <= 1e-5
    # the same call through mha (sm_scale explicit) and the forced route
    got2 = A.mha(*(to_dev(x, device, torch.float32) for x in (q, k, v)), mask=CausalMask(), sm_scale=1 / 8)
    assert torch.equal(got, got2)
    got3 = A.hip_attention_or_none(*(to_dev(x, device, torch.float32) for x in (q, k, v)),
                                   mask=CausalMask(), bias=None, dropout_rate=0.0, sm_scale=1 / 8)
    assert torch.equal(got, got3)


def test_config2_shape_reduced_bf16(device):
    from probjax_amd import attention as A
    from probjax_amd.masks import CausalMask

    q, k, v = (oracle.round_bf16(x) for x in rng_normal(1, (1, 1024, 2, 128), (1, 1024, 2, 128), (1, 1024, 2, 128)))
    want = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(128))
    got = A.flex_attention(*(_bf(x, device) for x in (q, k, v)), mask=CausalMask())
    assert max_abs(to_np(got), want) <= 2e-2


def test_config3_gqa_decode_kvlen_dispatches_splitkv(device, monkeypatch):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H
    from probjax_amd.masks import KVLenMask

    lengths = np.array([2048, 700, 1], np.int32)
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(2, (3, 1, 32, 128), (3, 2048, 8, 128), (3, 2048, 8, 128)))
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=1 / math.sqrt(128))
    calls = []
    real = H.splitkv_decode
    monkeypatch.setattr(H, "splitkv_decode", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    got = A.flex_attention(*(_bf(x, device) for x in (q, k, v)),
                           mask=KVLenMask(torch.from_numpy(lengths).to(device)), enable_gqa=True)
    assert calls, "a decode-shaped call should run the split-KV kernel"
    assert max_abs(to_np(got), want) <= 2e-2


def test_cached_decode_key_padding_mask_dispatches_splitkv(device, monkeypatch):
    """MultiHeadAttention's cached decode step (layers/attention.py:612-675)
    builds KeyPaddingMask(full(B, index + 1)) for one query row; the route
    takes it as per-batch KV lengths and runs the split-KV kernel."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H
    from probjax_amd.masks import KeyPaddingMask

    lengths = np.full(2, 1500, np.int32)
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(7, (2, 1, 16, 128), (2, 2048, 16, 128), (2, 2048, 16, 128)))
    want = oracle.xla_attention(q, k, v, mask=oracle.KeyPaddingMask(lengths), sm_scale=1 / math.sqrt(128))
    calls = []
    real = H.splitkv_decode
    monkeypatch.setattr(H, "splitkv_decode", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    got = A.flex_attention(*(_bf(x, device) for x in (q, k, v)),
                           mask=KeyPaddingMask(torch.from_numpy(lengths).to(device)))
    assert calls, "a one-row KeyPaddingMask call should run the split-KV kernel"
    assert max_abs(to_np(got), want) <= 2e-2


def test_config4_bias_and_padding_mask(device):
    import torch
    from probjax_amd import attention as A
    from probjax_amd.masks import DenseBias, KVLenMask

    b, l, h, d = 2, 512, 4, 64
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(3, (b, l, h, d), (b, l, h, d), (b, l, h, d)))
    (bias,) = rng_normal(4, (h, l, l), scale=0.5)
    lengths = np.array([l - 51, l - 40], np.int32)
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths),
                                bias=oracle.DenseBias(bias[None]), sm_scale=1 / 8)
    got = A.flex_attention(*(_bf(x, device) for x in (q, k, v)),
                           mask=KVLenMask(torch.from_numpy(lengths).to(device)),
                           bias=DenseBias(to_dev(bias[None], device, torch.float32)))
    assert max_abs(to_np(got), want) <= 2e-2


def test_config5_mla_absorbed_with_rope(device):
    """q = [q_nope W_UK | rope(q_pe)], cache = [c_kv | rope(k_pe)], sm_scale
    1/sqrt(128 + 64), output sliced to the latent width then W_UV."""
    import torch
    from probjax_amd import attention as A

    B, H, S, R, dn, dr = 2, 16, 600, 512, 128, 64
    c_kv, k_pe, q_nope, q_pe = rng_normal(5, (B, S, R), (B, S, dr), (B, 1, H, dn), (B, 1, H, dr))
    w_uk, w_uv = rng_normal(6, (H, dn, R), (H, dn, R), scale=0.02)
    k_rot = oracle.apply_rotary(k_pe, np.arange(S))
    q_rot = oracle.apply_rotary(q_pe, np.array([S]))
    q_cat = oracle.round_bf16(np.concatenate([np.einsum("bqhd,hdr->bqhr", q_nope, w_uk), q_rot], -1))
    cache = oracle.round_bf16(np.concatenate([c_kv, k_rot], -1))
    scale = 1 / math.sqrt(dn + dr)
    o_lat = oracle.xla_mla(q_cat, cache, sm_scale=scale)[..., :R]
    got = A.mla(_bf(q_cat, device), _bf(cache, device), sm_scale=scale, v_dim=R)
    assert max_abs(to_np(got), o_lat) <= 2e-2
    # the API-exact output (all 576 columns) agrees on the shared columns
    full = A.mla(_bf(q_cat, device), _bf(cache, device), sm_scale=scale)
    assert full.shape[-1] == 576
    assert max_abs(to_np(full)[..., :R], to_np(got)) <= 1e-2
    out = np.einsum("bqhr,hdr->bqhd", to_np(got), w_uv)
    want = np.einsum("bqhr,hdr->bqhd", o_lat, w_uv)
    assert max_abs(out, want) <= 2e-2


def test_dot_product_attention_leading_batch_dims_and_gqa(device):
    from probjax_amd import attention as A

    q, k, v = (oracle.round_bf16(x) for x in rng_normal(7, (2, 3, 64, 4, 64), (2, 3, 64, 2, 64), (2, 3, 64, 2, 64)))
    got = A.dot_product_attention(*(_bf(x, device) for x in (q, k, v)))
    want = oracle.xla_attention(q.reshape(6, 64, 4, 64), k.reshape(6, 64, 2, 64), v.reshape(6, 64, 2, 64),
                                sm_scale=1 / 8).reshape(2, 3, 64, 4, 64)
    assert tuple(got.shape) == (2, 3, 64, 4, 64)
    assert max_abs(to_np(got), want) <= 2e-2


def test_route_falls_through_for_unsupported_on_device(device):
    import torch
    from probjax_amd import attention as A

    q = torch.zeros(1, 16, 2, 300, dtype=torch.bfloat16, device=device)  # head_dim 300 > 256
    assert A.hip_attention_or_none(q, q, q, mask=None, bias=None, dropout_rate=0.0, sm_scale=0.1) is None
    with pytest.raises(ValueError, match="head_dim 300"):
        A.mha(q, q, q)
    q32 = torch.zeros(1, 16, 2, 260, dtype=torch.float32, device=device)  # fp32 kernels stop at 256
    assert A.hip_attention_or_none(q32, q32, q32, mask=None, bias=None, dropout_rate=0.0, sm_scale=0.1) is None
    with pytest.raises(ValueError, match="head_dim 260"):
        A.mha(q32, q32, q32)
