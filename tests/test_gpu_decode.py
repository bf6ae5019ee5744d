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
@pytest.mark.parametrize("streamed", ["0", "1"])
def test_splitkv_decode_matches_oracle(device, monkeypatch, streamed, b, lq, s, hq, hkv, d, lengths, chunk):
    """Both GQA decode kernels: the one that leaves K/V cacheable and the
    streaming one (non-temporal loads, K staged through LDS), which the
    capacity rule picks past 768 MiB of K/V and PJX_DECODE_STREAM forces."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import splitkv_decode

    monkeypatch.setenv("PJX_DECODE_STREAM", streamed)

    q, k, v = (oracle.round_bf16(x) for x in rng_normal(10, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, d)))
    scale = 1.0 / math.sqrt(d)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="tiled",
                                          return_lse=True)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = splitkv_decode(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)), sm_scale=scale,
                              kv_lengths=L, chunk=chunk, return_lse=True)
    launched = native.last_launches()
    torch.cuda.synchronize()
    if b > 0:
        assert launched[0].startswith("gqa_decode_kernel<Bf16Fmt") and launched[0].endswith(
            ", true>" if streamed == "1" else ", false>"), launched
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
        (2, 1, 16, 900, 256, 256, [900, 33], 0),             # rank 256
        (3, 1, 8, 500, 64, 64, [500, 0, 64], 128),           # rank 64, an empty sequence
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


# Head dims beyond 128, Dv != D and row groups: (dtype, B, Lq, S, Hq, Hkv, D, Dv,
# lengths, chunk, launched instance).  A row group holds up to 64 packed rows
# (4 blocks of 16) in bf16 / fp16 at D, Dv <= 128, else 32 (2 blocks); more
# rows run as several row groups over the same keys (the reference's row
# blocks, attention_splitkv.py:155-172).
WIDE_CASES = [
    ("bf16", 2, 1, 1500, 8, 2, 256, 256, [1500, 333], 256, "gqa_decode_kernel<Bf16Fmt, 256, 256, 1, false>"),
    ("bf16", 3, 2, 1100, 32, 2, 256, 256, [1100, 0, 517], 0, "gqa_decode_kernel<Bf16Fmt, 256, 256, 2, false>"),
    ("f16", 2, 1, 900, 16, 4, 256, 128, [900, 129], 128, "gqa_decode_kernel<F16Fmt, 256, 128, 1, false>"),
    ("bf16", 2, 3, 800, 8, 1, 128, 64, [800, 64], 128, "gqa_decode_kernel<Bf16Fmt, 128, 64, 2, false>"),
    ("bf16", 2, 1, 1000, 8, 2, 64, 128, None, 256, "gqa_decode_kernel<Bf16Fmt, 64, 128, 1, false>"),
    ("bf16", 1, 2, 700, 16, 1, 64, 256, [650], 128, "gqa_decode_kernel<Bf16Fmt, 64, 256, 2, false>"),
    # row groups: 128 rows (two groups of 64), 96 rows (a partial second group)
    ("bf16", 2, 16, 1200, 16, 2, 128, 128, [1200, 301], 0, "gqa_decode_kernel<Bf16Fmt, 128, 128, 4, false>"),
    ("f16", 2, 3, 1000, 64, 2, 64, 64, [1000, 1], 256, "gqa_decode_kernel<F16Fmt, 64, 64, 4, false>"),
    # D = 256 with 72 rows: three groups of 32, the last partial
    ("bf16", 2, 9, 600, 16, 2, 256, 256, [600, 300], 128, "gqa_decode_kernel<Bf16Fmt, 256, 256, 2, false>"),
    # fp32: groups of 32 rows; D / Dv up to 256
    ("f32", 2, 6, 900, 16, 2, 128, 128, [900, 450], 256, "gqa_decode_f32_kernel<128, 128, 2>"),
    ("f32", 2, 1, 1300, 8, 2, 256, 256, [1300, 77], 0, "gqa_decode_f32_kernel<256, 256, 1>"),
    ("f32", 2, 2, 700, 20, 2, 256, 64, [700, 0], 128, "gqa_decode_f32_kernel<256, 64, 2>"),
    ("f32", 1, 1, 1000, 8, 1, 64, 128, None, 256, "gqa_decode_f32_kernel<64, 128, 1>"),
]


@pytest.mark.parametrize("dtype,b,lq,s,hq,hkv,d,dv,lengths,chunk,inst", WIDE_CASES)
def test_splitkv_decode_head_dims_and_row_groups(device, dtype, b, lq, s, hq, hkv, d, dv, lengths, chunk, inst):
    """Split-KV decode at D, Dv in {64, 128, 256} (Dv != D included) and past
    64 packed rows (32 in fp32), against the oracle: bf16 / fp16 within 2e-2
    of the fp32 oracle on the same rounded inputs (fp16 also closer than the
    bf16-mode oracle), fp32 within 1e-5 of the float64 oracle; LSE +inf
    exactly for empty sequences.  The launched instance is asserted."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import splitkv_decode

    rows = (hq // hkv) * lq
    print(f"split-KV {dtype} B={b} Lq={lq} S={s} Hq={hq} Hkv={hkv} D={d} Dv={dv} rows={rows} -> {inst}", flush=True)
    q, k, v = rng_normal(13, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, dv))
    low = dtype != "f32"
    if low:
        rnd = oracle.round_bf16 if dtype == "bf16" else oracle.round_f16
        q, k, v = (rnd(x) for x in (q, k, v))
    scale = 1.0 / math.sqrt(d)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="tiled", return_lse=True,
                                          dtype=dtype, compute_dtype=np.float32 if low else np.float64)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    got, lse = splitkv_decode(*(to_dev(x, device, tdt) for x in (q, k, v)), sm_scale=scale,
                              kv_lengths=L, chunk=chunk, return_lse=True)
    launched = native.last_launches()
    torch.cuda.synchronize()
    assert launched[0] == inst, launched
    assert got.shape == (b, lq, hq, dv) and got.dtype == tdt
    err = max_abs(to_np(got), want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= (BF16_TOL if low else 1e-5)
    if dtype == "f16":
        want_bf = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="tiled", dtype="bf16")
        d_got = np.sqrt(np.mean((to_np(got).astype(np.float64) - want) ** 2))
        d_bf = np.sqrt(np.mean((want_bf.astype(np.float64) - want) ** 2))
        assert d_got <= 0.5 * d_bf
    lse = to_np(lse)
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= (1e-3 if low else 1e-5)


@pytest.mark.parametrize("dtype,b,lq,s,hq,hkv,d,dv,lengths,chunk,inst", [c for c in WIDE_CASES if c[0] != "f32"])
def test_splitkv_decode_streamed_head_dims_and_row_groups(device, monkeypatch, dtype, b, lq, s, hq, hkv, d, dv,
                                                          lengths, chunk, inst):
    """The streaming GQA decode instances at every head-dim pair and row-block
    count of the cases above (forced with PJX_DECODE_STREAM=1), to the same
    bar against the oracle."""
    monkeypatch.setenv("PJX_DECODE_STREAM", "1")
    test_splitkv_decode_head_dims_and_row_groups(device, dtype, b, lq, s, hq, hkv, d, dv, lengths, chunk,
                                                 inst.replace(", false>", ", true>"))


@pytest.mark.parametrize(
    "b,lq,h,s,r,dv,lengths,chunk",
    [
        (2, 1, 32, 700, 576, 512, [700, 333], 0),           # 2 row groups of 16
        (3, 1, 128, 600, 576, 512, [600, 0, 65], 128),       # 8 row groups, an empty sequence
        (2, 2, 40, 500, 512, 512, None, 128),                # Lq = 2: 80 folded rows, t*H + h
        (2, 1, 20, 800, 128, 128, [800, 17], 0),             # 20 rows: a partial second group
    ],
)
@pytest.mark.parametrize("streamed", ["0", "1"])
def test_mla_decode_row_groups(device, monkeypatch, streamed, b, lq, h, s, r, dv, lengths, chunk):
    """The latent decode past 16 folded rows: each 16 rows form a row group
    streaming the cache chunk by chunk (the reference's mla takes any head
    count, latent_attention.py:636-766), against the oracle within 2e-2; both
    the cacheable kernel and the streaming one (non-temporal loads), which the
    capacity rule picks past 512 MiB of latent and PJX_DECODE_STREAM forces."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import mla_decode

    monkeypatch.setenv("PJX_DECODE_STREAM", streamed)
    print(f"MLA decode B={b} Lq={lq} H={h} S={s} R={r} Dv={dv} rows={lq * h}", flush=True)
    q, cache = (oracle.round_bf16(x) for x in rng_normal(14, (b, lq, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    mask = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, mask=mask, sm_scale=scale, strategy="tiled",
                                          return_lse=True)
    want = want[..., :dv]
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    got, lse = mla_decode(to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16),
                          sm_scale=scale, v_dim=dv, kv_lengths=L, chunk=chunk, return_lse=True)
    launched = native.last_launches()
    torch.cuda.synchronize()
    assert launched[0] == f"mla_decode_kernel<Bf16Fmt, {r}, {dv}, {'true' if streamed == '1' else 'false'}>", launched
    err = max_abs(to_np(got), want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= BF16_TOL
    lse = to_np(lse)
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-3


def test_splitkv_forward_head_dims(device):
    """probjax's splitkv_forward with qk head dim 192 and value head dim 96
    (padded to the kernel's 256 / 128) matches the oracle at the true dims;
    mha sends a D = 192 decode step to the split-KV kernel."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import native

    b, lq, s, hq, hkv, d, dv = 2, 1, 2048, 16, 4, 192, 96
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(15, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, dv)))
    lengths = np.array([2048, 1111], np.int32)
    scale = 1.0 / math.sqrt(d)
    want, want_lse = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=scale, return_lse=True)
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    L = torch.from_numpy(lengths).to(device)
    got, lse = A.splitkv_forward(tq, tk, tv, sm_scale=scale, kv_lengths=L, return_lse=True)
    torch.cuda.synchronize()
    assert got.shape == (b, lq, hq, dv)
    assert max_abs(to_np(got), want) <= BF16_TOL
    assert max_abs(to_np(lse), want_lse) <= 1e-3
    # mha (Dv = D): the decode route pads 192 to 256
    v2 = oracle.round_bf16(rng_normal(16, (b, s, hkv, d))[0])
    want2 = oracle.xla_attention(q, k, v2, mask=oracle.KVLenMask(lengths), sm_scale=scale)
    from probjax_amd.masks import KVLenMask

    assert A.use_splitkv(tq, tk, mask=KVLenMask(L))
    out = A.mha(tq, tk, to_dev(v2, device, torch.bfloat16), mask=KVLenMask(L), sm_scale=scale)
    launched = native.last_launches()
    torch.cuda.synchronize()
    assert launched[0] == "gqa_decode_kernel<Bf16Fmt, 256, 256, 1, false>", launched
    assert max_abs(to_np(out), want2) <= BF16_TOL


@pytest.mark.parametrize("r,dv,want_inst", [(200, 150, "mla_decode_kernel<Bf16Fmt, 256, 256, false>"),
                                            (576, 300, "mla_decode_kernel<Bf16Fmt, 576, 512, false>"),
                                            (40, 40, "mla_decode_kernel<Bf16Fmt, 64, 64, false>")])
def test_mla_decode_route_pads_rank(device, r, dv, want_inst):
    """Absorbed mla decode steps at a latent width between the kernel ranks
    zero-pad q and the cache to the next rank (zero features change no score)
    and slice the output columns, keeping the split-KV latent kernel."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import native
    from probjax_amd.masks import KVLenMask

    b, h, s = 2, 16, 700
    q, cache = (oracle.round_bf16(x) for x in rng_normal(17, (b, 1, h, r), (b, s, r)))
    lengths = np.array([700, 255], np.int32)
    scale = 1.0 / math.sqrt(192)
    shared = cache[:, :, None, :]
    want = oracle.xla_attention(q, shared, shared, mask=oracle.KVLenMask(lengths), sm_scale=scale)[..., :dv]
    out = A.mla(to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16), sm_scale=scale,
                v_dim=dv, mask=KVLenMask(torch.from_numpy(lengths).to(device)))
    launched = native.last_launches()
    torch.cuda.synchronize()
    assert launched[0] == want_inst, launched
    assert out.shape == (b, 1, h, dv)
    assert max_abs(to_np(out), want) <= BF16_TOL


@pytest.mark.parametrize("dtype,d,dv,lq", [("bf16", 128, 128, 1), ("f16", 64, 256, 2), ("bf16", 256, 64, 5)])
def test_streamed_decode_is_bitwise_equal(device, monkeypatch, dtype, d, dv, lq):
    """The streaming and the ordinary GQA decode kernels compute the same
    products in the same order: outputs and LSE are bitwise equal."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import splitkv_decode

    b, s, hq, hkv = 3, 1700, 16, 2
    tdt = torch.bfloat16 if dtype == "bf16" else torch.float16
    q, k, v = (to_dev(x, device, tdt) for x in rng_normal(17, (b, lq, hq, d), (b, s, hkv, d), (b, s, hkv, dv)))
    L = torch.tensor([1700, 999, 37], dtype=torch.int32, device=device)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("PJX_DECODE_STREAM", flag)
        out[flag] = splitkv_decode(q, k, v, sm_scale=0.1, kv_lengths=L, chunk=256, return_lse=True)
        launched = native.last_launches()
        assert launched[0].endswith(", true>" if flag == "1" else ", false>"), launched
    torch.cuda.synchronize()
    assert torch.equal(out["0"][0], out["1"][0])
    assert torch.equal(out["0"][1], out["1"][1])


def test_streamed_mla_decode_is_bitwise_equal(device, monkeypatch):
    """The streaming and the cacheable latent decode kernels differ only in the
    load hint: outputs and LSE are bitwise equal."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import mla_decode

    b, s, h, r, dv = 3, 1300, 24, 576, 512
    q, cache = (to_dev(x, device, torch.bfloat16) for x in rng_normal(18, (b, 1, h, r), (b, s, r)))
    L = torch.tensor([1300, 640, 5], dtype=torch.int32, device=device)
    out = {}
    for flag in ("0", "1"):
        monkeypatch.setenv("PJX_DECODE_STREAM", flag)
        out[flag] = mla_decode(q, cache, sm_scale=0.07, v_dim=dv, kv_lengths=L, return_lse=True)
        launched = native.last_launches()
        assert launched[0] == f"mla_decode_kernel<Bf16Fmt, {r}, {dv}, {'true' if flag == '1' else 'false'}>", launched
    torch.cuda.synchronize()
    assert torch.equal(out["0"][0], out["1"][0])
    assert torch.equal(out["0"][1], out["1"][1])


@pytest.mark.parametrize("r,lq,h", [(256, 2, 40), (128, 2, 40), (64, 2, 40), (256, 1, 64)])
def test_mla_decode_shared_cu_repeatable(device, r, lq, h):
    """Ranks <= 256 run several latent-decode workgroups per CU, whose waves
    share each SIMD's matrix pipe.  With 128-key chunks (two tiles per item)
    and several row groups, scores once reached their LDS exchange before the
    last MFMA had finished with them: wrong terms for a few rows that changed
    from run to run.  Four calls on the same inputs must agree bitwise and
    with the oracle."""
    import torch
    from probjax_amd.hip_attention import mla_decode

    b, s, chunk = 3, 2372, 128
    print(f"latent decode repeat R={r} Lq={lq} H={h} S={s} chunk={chunk}", flush=True)
    q, cache = (oracle.round_bf16(x) for x in rng_normal(404, (b, lq, h, r), (b, s, r)))
    scale = 1.0 / math.sqrt(192)
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, sm_scale=scale, strategy="dense", dtype="bf16",
                                          return_lse=True)
    qd, cd = to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16)
    outs = [mla_decode(qd, cd, sm_scale=scale, v_dim=r, chunk=chunk, return_lse=True) for _ in range(4)]
    torch.cuda.synchronize()
    for o, lse in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(lse, outs[0][1])
    assert max_abs(to_np(outs[0][0]), want) <= BF16_TOL
    assert max_abs(to_np(outs[0][1]), want_lse) <= 1e-4
