"""Parity at the full sizes of the head-dim-256 and absorbed-latent bench
workloads: C2W / C2WB (bf16 causal B=2, H=16, L=4096, D=256, forward and
backward) and C5A / C5AB (absorbed latent, bf16 causal B=1, H=16, L=4096,
R=576, v_dim 512, forward and backward).

Every batch, head and row is compared with the oracle (``xla_attention`` /
``oracle.backward.attention_backward`` in fp32 on the same bf16 inputs; for
the latent, K = V = the cache broadcast to every head and dcache = dK + dV, as
in probjax's custom VJP, kernels/latent_attention.py:752-766).  The kernels'
backward takes the kernels' own forward output and LSE, as the autograd path
does.  Tolerances: outputs max-abs <= 2e-2, LSE <= 1e-2; gradients within
probjax's gradient tolerance (atol 2e-2, rtol 1e-2, tests/test_attention.py:
597-626) with atol scaled by max(1, max|ref| / 4), since dK, dV and dcache sum
4096 query rows (and 16 heads for dcache).
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, to_dev, to_np

pytestmark = pytest.mark.gpu


def _bf16_inputs(seed, *shapes):
    rng = np.random.default_rng(seed)
    return [oracle.round_bf16(rng.standard_normal(s, dtype=np.float32)) for s in shapes]


def _check_grad(name, got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    atol = 2e-2 * max(1.0, float(np.max(np.abs(want))) / 4.0)
    err = np.abs(got - want)
    bad = err > atol + 1e-2 * np.abs(want)
    print(f"  {name}: max err {err.max():.3e} (atol {atol:.3e}), rms {np.sqrt(np.mean(err ** 2)):.3e}", flush=True)
    assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.size} outside tolerance, max err {err.max():.3e}"


def test_c2w_forward_and_backward_full_size(device):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd, flash_attention_fwd

    B, L, H, D = 2, 4096, 16, 256
    scale = 1.0 / math.sqrt(D)
    q, k, v, do = _bf16_inputs(21, (B, L, H, D), (B, L, H, D), (B, L, H, D), (B, L, H, D))
    print(f"C2W/C2WB full size: B={B} L={L} H={H} D={D} causal", flush=True)
    tq, tk, tv, tdo = (to_dev(x, device, torch.bfloat16) for x in (q, k, v, do))
    out, lse = flash_attention_fwd(tq, tk, tv, sm_scale=scale, causal=True, return_lse=True)
    dq, dk, dv = flash_attention_bwd(tq, tk, tv, out, tdo, lse, sm_scale=scale, causal=True)
    torch.cuda.synchronize()
    out, lse, dq, dk, dv = (to_np(t) for t in (out, lse, dq, dk, dv))
    for b in range(B):
        sl = slice(b, b + 1)
        want, want_lse = oracle.xla_attention(q[sl], k[sl], v[sl], mask=oracle.CausalMask(), sm_scale=scale,
                                              return_lse=True)
        err = max_abs(out[sl], want)
        print(f"  batch {b}: output max-abs {err:.3e}", flush=True)
        assert err <= 2e-2
        assert max_abs(lse[sl], want_lse) <= 1e-2
        gq, gk, gv = attention_backward(q[sl], k[sl], v[sl], want, do[sl], want_lse, mask=oracle.CausalMask(),
                                        sm_scale=scale, dtype="f32", compute_dtype=np.float32)
        _check_grad(f"batch {b} dq", dq[sl], gq)
        _check_grad(f"batch {b} dk", dk[sl], gk)
        _check_grad(f"batch {b} dv", dv[sl], gv)
    # causal row 0 attends to key 0 only
    np.testing.assert_array_equal(out[:, 0], v[:, 0])


def test_c5a_forward_and_backward_full_size(device):
    import torch
    from probjax_amd.hip_attention import mla_bwd, mla_fwd

    B, L, H, R, DV = 1, 4096, 16, 576, 512
    scale = 1.0 / math.sqrt(192)
    q, cache, do = _bf16_inputs(22, (B, L, H, R), (B, L, R), (B, L, H, DV))
    print(f"C5A/C5AB full size: B={B} L={L} H={H} R={R} v_dim={DV} causal", flush=True)
    tq, tc, tdo = to_dev(q, device, torch.bfloat16), to_dev(cache, device, torch.bfloat16), to_dev(do, device, torch.bfloat16)
    out, lse = mla_fwd(tq, tc, sm_scale=scale, v_dim=DV, causal=True, return_lse=True)
    dq, dc = mla_bwd(tq, tc, out, tdo, lse, sm_scale=scale, causal=True)
    torch.cuda.synchronize()
    out, lse, dq, dc = (to_np(t) for t in (out, lse, dq, dc))
    shared = cache[:, :, None, :]
    want, want_lse = oracle.xla_attention(q, shared, shared, mask=oracle.CausalMask(), sm_scale=scale,
                                          return_lse=True)
    err = max_abs(out, want[..., :DV])
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= 2e-2
    assert max_abs(lse, want_lse) <= 1e-2
    # the output keeps the first DV columns: their gradient, zeros beyond
    dop = np.concatenate([do, np.zeros(do.shape[:-1] + (R - DV,), np.float32)], axis=-1)
    gq, gk, gv = attention_backward(q, shared, shared, want, dop, want_lse, mask=oracle.CausalMask(),
                                    sm_scale=scale, dtype="f32", compute_dtype=np.float32)
    _check_grad("dq", dq, gq)
    _check_grad("dcache", dc, (np.asarray(gk, np.float64) + np.asarray(gv, np.float64))[:, :, 0])
