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
        # longest-first item order: equal remainders (ties), exact multiples of
        # the chunk, lengths past the cache and negative lengths (clamped)
        (12, 1, 640, 8, 2, 64, [640, 600, 600, 128, 129, 0, -3, 9999, 600, 256, 1, 383], 128),
        # more sequences than the in-kernel scheduler orders: chunk-major order
        (300, 1, 256, 4, 1, 64, [(37 * i) % 300 - 20 for i in range(300)], 128),
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


@pytest.mark.parametrize(
    "b,lq,h,s,r,dv,lengths,chunk",
    [
        (2, 1, 16, 700, 576, 512, None, 0),
        (2, 1, 16, 700, 576, 576, None, 0),
        (3, 1, 16, 1000, 576, 512, [1, 63, 1000], 192),     # 3-tile chunks, partial last tiles
        (4, 1, 8, 513, 576, 512, [0, 64, 65, 513], 64),      # empty sequence, one-tile chunks, 8 rows
        (2, 2, 4, 300, 512, 512, [300, 129], 128),           # Lq = 2: rows fold as t*H + h
        (2, 1, 16, 2000, 512, 512, None, 0),
        (2, 1, 16, 777, 128, 128, [777, 5], 0),
        (1, 1, 16, 4096, 576, 512, [4096], 8192),            # one chunk: the chunk kernel writes the output
        (5, 1, 3, 257, 576, 576, [257, 256, 2, 128, 129], 128),  # 3 rows
        (6, 1, 4, 600, 512, 512, [600, 320, 320, 5, -1, 700], 128),  # ties, clamped lengths
    ],
)
def test_mla_decode_matches_oracle(device, b, lq, h, s, r, dv, lengths, chunk):
    import torch
    from probjax_amd.hip_attention import mla_decode

    q, cache = (oracle.round_bf16(x) for x in rng_normal(11, (b, lq, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, mask=mask, sm_scale=scale, strategy="tiled",
                                          return_lse=True)
    want = want[..., :dv]
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = mla_decode(to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16),
                          sm_scale=scale, v_dim=dv, kv_lengths=L, chunk=chunk, return_lse=True)
    torch.cuda.synchronize()
    assert max_abs(to_np(got), want) <= BF16_TOL
    lse = to_np(lse)
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-3


@pytest.mark.parametrize(
    "dtype,b,lq,s,hq,hkv,d,lengths,chunk",
    [
        ("bf16", 2, 2, 2000, 16, 2, 128, [2000, 999], 0),       # G = 8, Lq = 2: 16 rows
        ("bf16", 2, 4, 1500, 32, 4, 128, [1500, 700], 256),     # G = 8, Lq = 4: 32 rows (speculative decode)
        ("bf16", 3, 8, 1200, 16, 2, 128, [1200, 1, 0], 0),      # G = 8, Lq = 8: 64 rows, empty sequence
        ("bf16", 2, 5, 900, 24, 2, 64, [900, 450], 128),        # 60 rows: a partial last row block
        ("f32", 3, 1, 1000, 8, 2, 128, [1, 500, 1000], 0),
        ("f32", 2, 4, 1500, 32, 4, 128, [1500, 700], 256),      # 32 rows
        ("f32", 2, 3, 700, 10, 2, 64, [700, 0], 128),           # 15 rows, empty sequence
        ("f32", 2, 2, 3000, 16, 1, 128, None, 512),             # 32 rows, no lengths, merge
    ],
)
def test_splitkv_decode_wide_rows_and_fp32(device, dtype, b, lq, s, hq, hkv, d, lengths, chunk):
    """More than 16 packed rows per KV head (up to the reference's 64,
    attention_splitkv.py:155-170) and fp32 inputs (full fp32 products):
    bf16 within 2e-2 of the fp32 oracle, fp32 within 1e-5 of the float64
    oracle; empty rows give LSE = +inf."""
    import torch
    from probjax_amd.hip_attention import splitkv_decode

    print(f"split-KV {dtype} B={b} Lq={lq} S={s} Hq={hq} Hkv={hkv} D={d} rows={(hq // hkv) * lq}", flush=True)
    q, k, v = rng_normal(11, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, d))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v = (oracle.round_bf16(x) for x in (q, k, v))
    scale = 1.0 / math.sqrt(d)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="tiled", return_lse=True,
                                          compute_dtype=np.float32 if bf16 else np.float64)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    tdt = torch.bfloat16 if bf16 else torch.float32
    got, lse = splitkv_decode(*(to_dev(x, device, tdt) for x in (q, k, v)), sm_scale=scale,
                              kv_lengths=L, chunk=chunk, return_lse=True)
    torch.cuda.synchronize()
    assert got.dtype == tdt
    err = max_abs(to_np(got), want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= (BF16_TOL if bf16 else 1e-5)
    lse = to_np(lse)
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= (1e-3 if bf16 else 1e-5)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_wide_and_fp32_decode_route_to_splitkv(device, monkeypatch, dtype):
    """mha's use_splitkv rule (Lq <= 64, Lkv >= 1024, kernels/attention.py:
    2653-2689) sends a GQA-8 speculative step (Lq = 4, 32 rows) and an fp32
    decode to the split-KV kernel, and the result matches the oracle."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as hip
    from probjax_amd.masks import KVLenMask

    calls = []
    orig = hip.splitkv_decode

    def spy(*a, **k):
        calls.append(1)
        return orig(*a, **k)

    monkeypatch.setattr(hip, "splitkv_decode", spy)
    b, lq, s, hq, hkv, d = 2, 4, 2048, 32, 4, 128
    q, k, v = rng_normal(12, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, d))
    bf16 = dtype == "bf16"
    if bf16:
        q, k, v = (oracle.round_bf16(x) for x in (q, k, v))
    lengths = np.array([2048, 1500], np.int32)
    tdt = torch.bfloat16 if bf16 else torch.float32
    assert A.use_splitkv(to_dev(q, device, tdt), to_dev(k, device, tdt), mask=KVLenMask(lengths))
    out = A.mha(*(to_dev(x, device, tdt) for x in (q, k, v)), mask=KVLenMask(torch.from_numpy(lengths).to(device)),
                sm_scale=1 / math.sqrt(d))
    assert calls == [1]
    want = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=1 / math.sqrt(d),
                                compute_dtype=np.float32 if bf16 else np.float64)
    assert max_abs(to_np(out), want) <= (BF16_TOL if bf16 else 1e-5)
