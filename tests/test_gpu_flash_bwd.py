"""Parity of the HIP flash-attention backward with the CPU oracle.

The kernels get the oracle forward's output and LSE, so the comparison
isolates the backward: dq, dk, dv against ``oracle.backward.attention_backward``
in bf16 mode (same bf16 roundings of P and dS), within probjax's own gradient
tolerance (tests/test_attention.py:597-626: atol 2e-2, rtol 1e-2).
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def _mask(causal, lengths):
    m = oracle.CausalMask() if causal else None
    if lengths is not None:
        kl = oracle.KVLenMask(np.array(lengths, np.int32))
        m = kl if m is None else m & kl
    return m


def _check(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bad = err > ATOL + RTOL * np.abs(want)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside atol {ATOL} rtol {RTOL}; "
        f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    )


CASES = [
    # B, Lq, Lk, Hq, Hkv, D, causal, lengths, bias_shape
    (1, 256, 256, 4, 4, 128, True, None, None),
    (2, 300, 300, 4, 2, 128, True, None, None),             # GQA, partial tiles
    (2, 200, 333, 8, 2, 64, False, [333, 150], None),       # Lq != Lk, ragged lengths
    (1, 512, 512, 4, 1, 128, True, [400], None),            # MQA: 4 heads per KV head
    (2, 256, 256, 4, 4, 64, False, [256, 200], (1, 4)),     # dense bias per head
    (1, 192, 192, 4, 2, 128, True, None, (1, 1)),           # broadcast bias, causal
    (2, 130, 130, 2, 2, 128, False, [0, 100], None),        # every row of batch 0 empty
    (1, 100, 300, 2, 1, 64, True, None, None),              # causal with Lq < Lk
    (1, 1024, 1024, 2, 2, 128, True, None, None),           # many tiles per workgroup
]


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,D,causal,lengths,bias_shape", CASES)
def test_flash_bwd_bf16_matches_oracle(device, B, Lq, Lk, Hq, Hkv, D, causal, lengths, bias_shape):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    print(f"case B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} causal={causal} "
          f"lengths={lengths} bias={bias_shape}", flush=True)
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(20, (B, Lq, Hq, D), (B, Lk, Hkv, D),
                                                           (B, Lk, Hkv, D), (B, Lq, Hq, D)))
    bias = None
    if bias_shape is not None:
        bias = rng_normal(21, (*bias_shape, Lq, Lk), scale=0.5)[0]
    scale = 1.0 / math.sqrt(D)
    mask = _mask(causal, lengths)
    db = oracle.DenseBias(bias) if bias is not None else None
    o, lse = oracle.xla_attention(q, k, v, mask=mask, bias=db, sm_scale=scale, strategy="dense",
                                  dtype="bf16", return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, bias=db, sm_scale=scale, dtype="bf16")

    bf = torch.bfloat16
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got = flash_attention_bwd(
        to_dev(q, device, bf), to_dev(k, device, bf), to_dev(v, device, bf), to_dev(o, device, bf),
        to_dev(do, device, bf), torch.from_numpy(lse).to(device), sm_scale=scale, causal=causal,
        kv_lengths=L, bias=bt,
    )
    torch.cuda.synchronize()
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        _check(to_np(g), w, name)
    if lengths is not None:
        # keys past each length: exactly zero gradients
        for b, n in enumerate(lengths):
            assert torch.count_nonzero(got[1][b, n:]) == 0 and torch.count_nonzero(got[2][b, n:]) == 0
            if n == 0:
                assert torch.count_nonzero(got[0][b]) == 0


def test_flash_bwd_static_lengths(device):
    """QKVLengthMask (q_valid / kv_valid): rows past q_valid get dq = 0."""
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    B, L, H, D = 1, 256, 2, 128
    qv, kvv = 200, 230
    q, k, v, do = (oracle.round_bf16(x) for x in rng_normal(22, (B, L, H, D), (B, L, H, D),
                                                           (B, L, H, D), (B, L, H, D)))
    scale = 1.0 / math.sqrt(D)
    mask = oracle.CausalMask() & oracle.QKVLengthMask(qv, kvv)
    o, lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, strategy="dense", dtype="bf16",
                                  return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, sm_scale=scale, dtype="bf16")
    bf = torch.bfloat16
    got = flash_attention_bwd(
        to_dev(q, device, bf), to_dev(k, device, bf), to_dev(v, device, bf), to_dev(o, device, bf),
        to_dev(do, device, bf), torch.from_numpy(lse).to(device), sm_scale=scale, causal=True,
        q_valid=qv, kv_valid=kvv,
    )
    torch.cuda.synchronize()
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        _check(to_np(g), w, name)
    assert torch.count_nonzero(got[0][:, qv:]) == 0
    assert torch.count_nonzero(got[1][:, kvv:]) == 0 and torch.count_nonzero(got[2][:, kvv:]) == 0


F32_CASES = [
    # B, Lq, Lk, Hq, Hkv, D, causal, lengths, bias_shape
    (1, 512, 512, 4, 4, 64, True, None, None),          # config 1's shape
    (2, 300, 300, 4, 2, 128, True, None, None),         # GQA, partial tiles
    (2, 200, 333, 4, 1, 64, False, [333, 0], (2, 1)),   # per-batch bias, empty batch, Lq != Lk
    (1, 160, 160, 2, 2, 128, False, [100], (1, 2)),
]


@pytest.mark.parametrize("B,Lq,Lk,Hq,Hkv,D,causal,lengths,bias_shape", F32_CASES)
def test_flash_bwd_f32_matches_float64_oracle(device, B, Lq, Lk, Hq, Hkv, D, causal, lengths, bias_shape):
    """fp32 gradients against the float64 oracle: max-abs <= 1e-5 * max(1, max|ref|)
    (the fp32 bar of 1e-5, scaled by the gradients' magnitude; the fp32 oracle
    itself sits ~2e-6 from float64 on these shapes)."""
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    print(f"case f32 B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} causal={causal} "
          f"lengths={lengths} bias={bias_shape}", flush=True)
    q, k, v, do = rng_normal(40, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D), (B, Lq, Hq, D))
    bias = None if bias_shape is None else rng_normal(41, (*bias_shape, Lq, Lk), scale=0.5)[0]
    scale = 1.0 / math.sqrt(D)
    mask = _mask(causal, lengths)
    db = oracle.DenseBias(bias) if bias is not None else None
    o, lse = oracle.xla_attention(q, k, v, mask=mask, bias=db, sm_scale=scale, strategy="dense",
                                  compute_dtype=np.float64, return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, bias=db, sm_scale=scale,
                              compute_dtype=np.float64)
    f = torch.float32
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got = flash_attention_bwd(
        to_dev(q, device, f), to_dev(k, device, f), to_dev(v, device, f), to_dev(o, device, f),
        to_dev(do, device, f), torch.from_numpy(lse).to(device), sm_scale=scale, causal=causal,
        kv_lengths=L, bias=bt,
    )
    torch.cuda.synchronize()
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        tol = 1e-5 * max(1.0, float(np.max(np.abs(w))))
        err = float(np.max(np.abs(to_np(g).astype(np.float64) - w)))
        assert err <= tol, f"{name}: max err {err:.3e} > {tol:.3e}"


@pytest.mark.parametrize("D,Hq,Hkv,L,causal", [(128, 16, 16, 2048, True), (64, 16, 4, 2048, True),
                                                (128, 8, 8, 2048, False), (128, 4, 2, 1000, True)])
def test_flash_bwd_small_grid_matches_large_grid(device, D, Hq, Hkv, L, causal):
    """Small grids (at most one workgroup per CU, or two with a causal mask) run
    the dQ and dK/dV kernels with two groups of waves per workgroup, each
    summing half of the tiles; the same inputs repeated over a batch large
    enough for the one-group forms give the same gradients to one bf16
    rounding (the same fp32 terms, summed in another order)."""
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd, flash_attention_fwd

    nkb = -(-L // 128)
    rep = (2 * 256) // (nkb * Hkv) + 1   # key blocks (and query tiles) above two per CU of a 256-CU device
    print(f"case D={D} Hq={Hq} Hkv={Hkv} L={L} causal={causal} rep={rep}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(31)
    bf = torch.bfloat16
    q, do = (torch.randn((1, L, Hq, D), generator=g, device=device).to(bf) for _ in range(2))
    k, v = (torch.randn((1, L, Hkv, D), generator=g, device=device).to(bf) for _ in range(2))
    scale = 1.0 / math.sqrt(D)
    o, lse = flash_attention_fwd(q, k, v, sm_scale=scale, causal=causal, return_lse=True)
    small = flash_attention_bwd(q, k, v, o, do, lse, sm_scale=scale, causal=causal)
    big_in = [x.expand(rep, *x.shape[1:]).contiguous() for x in (q, k, v, o, do, lse)]
    big = flash_attention_bwd(*big_in, sm_scale=scale, causal=causal)
    torch.cuda.synchronize()
    for name, gb, gs in zip(("dq", "dk", "dv"), big, small):
        a = gb.float()
        b = gs.float().expand_as(a)
        err = (a - b).abs()
        lim = 2.0 ** -7 * b.abs() + 1e-3 * b.abs().max()
        assert bool((err <= lim).all()), f"{name}: max err {err.max().item():.3e}"
