"""Parity of the HIP split-KV GQA decode and MLA decode with the CPU oracle."""

import math

import numpy as np
import pytest

import oracle
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

BF16_TOL = 2e-2


@pytest.mark.parametrize(
    "b,lq,s,hq,hkv,d,lengths,chunk",
    [
        (3, 1, 1000, 8, 2, 128, [1, 500, 1000], 0),
        (2, 1, 4096, 32, 8, 128, [4096, 2049], 0),
        (2, 2, 700, 8, 2, 128, None, 128),        # 6 chunks -> merge
        (2, 1, 300, 4, 4, 64, [300, 65], 128),
        (4, 1, 1500, 16, 1, 128, [0, 1, 129, 1500], 256),  # empty / single-key rows, 16 rows
        (1, 3, 2000, 20, 4, 64, [1999], 512),     # 15 rows, ragged tail per wave
        (3, 1, 8192, 32, 8, 128, [8192, 512, 7777], 0),
        (4, 1, 8192, 8, 2, 128, [1, 2, 3, 0], 128),      # chunks past every length: empty partials
        (16, 1, 300, 8, 2, 64, [7, 300, 1, 150, 299, 2, 64, 65, 0, 33, 120, 17, 280, 5, 9, 211], 128),
        (2, 1, 5000, 16, 4, 128, [5000, 4999], 0),
    ],
)
def test_splitkv_decode_matches_oracle(device, b, lq, s, hq, hkv, d, lengths, chunk):
    import torch
    from probjax_amd.hip_attention import splitkv_decode

    q, k, v = (oracle.round_bf16(x) for x in rng_normal(10, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, d)))
    scale = 1.0 / math.sqrt(d)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="tiled",
                                          return_lse=True)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = splitkv_decode(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)), sm_scale=scale,
                              kv_lengths=L, chunk=chunk, return_lse=True)
    torch.cuda.synchronize()
    assert max_abs(to_np(got), want) <= BF16_TOL
    lse = to_np(lse)
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))  # empty rows: +inf
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-3


@pytest.mark.parametrize("v_dim", [512, 576])
def test_mla_decode_matches_oracle(device, v_dim):
    import torch
    from probjax_amd.hip_attention import mla_decode

    b, h, s, r = 2, 16, 700, 576
    q, cache = (oracle.round_bf16(x) for x in rng_normal(11, (b, 1, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    want = oracle.xla_mla(q, cache, sm_scale=scale)[..., :v_dim]
    got = mla_decode(to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16),
                     sm_scale=scale, v_dim=v_dim)
    torch.cuda.synchronize()
    assert max_abs(to_np(got), want) <= BF16_TOL
