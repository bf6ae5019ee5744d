"""The backward's dS route (head dim 256), against the oracle and against the
two-kernel route on the same inputs.

With a workspace of ``pjx_flash_bwd_ds_workspace_size`` bytes, a call without
bias or score modifiers runs delta, the key-side kernel storing the rounded
dS, then dQ = dS K as one product per score (``wide_bwd_delta_kernel``,
``wide_bwd_dc_ds_kernel``, ``wide_bwd_dq_ds_kernel``); with the smaller
workspace the dQ kernel recomputes S and dP.  The launch log is asserted for
both routes.  Both form the same delta, the same 16-bit dS and the same fp32
sums in the same order, so their gradients are compared bitwise; each is also
held to the oracle with the gradient tolerance of the other backward tests
(probjax tests/test_attention.py:597-626: atol 2e-2 scaled by
max(1, max|ref| / 4), rtol 1e-2) against ``oracle.backward.attention_backward``
in the same 16-bit mode.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
FMT = {"bf16": "Bf16Fmt", "f16": "F16Fmt"}


def _round(x, dtype):
    return oracle.round_bf16(x) if dtype == "bf16" else oracle.round_f16(x)


def _tdt(dtype):
    import torch

    return torch.bfloat16 if dtype == "bf16" else torch.float16


def _check(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    atol = ATOL * max(1.0, float(np.max(np.abs(want), initial=0.0)) / 4.0)
    bad = err > atol + RTOL * np.abs(want)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside atol {atol:.3g} rtol {RTOL}; "
        f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    )


def _omask(causal, lengths, q_valid, kv_valid, Lq, Lk):
    m = oracle.CausalMask() if causal else None
    if lengths is not None:
        kl = oracle.KVLenMask(np.array(lengths, np.int32))
        m = kl if m is None else m & kl
    if q_valid is not None or kv_valid is not None:
        ql = oracle.QKVLengthMask(Lq if q_valid is None else q_valid, Lk if kv_valid is None else kv_valid)
        m = ql if m is None else m & ql
    return m


def _launched():
    from probjax_amd import native

    return native.last_launches()


# name: B, Lq, Lk, Hq, Hkv, causal, kv_lengths, q_valid, kv_valid
FLASH_CASES = {
    "causal_gqa": (1, 256, 256, 4, 2, True, None, None, None),
    "ragged_noncausal": (2, 200, 300, 4, 2, False, [300, 123], None, None),
    "causal_qvalid": (1, 300, 300, 8, 2, True, None, 250, None),
    "empty_sequence": (2, 130, 70, 2, 1, False, [70, 0], None, None),
    "many_heads": (1, 128, 192, 24, 24, True, None, None, None),
    "kv_valid": (2, 160, 260, 4, 4, False, None, None, 201),
    "one_query": (3, 1, 333, 8, 2, False, [333, 17, 200], None, None),
}


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("name", list(FLASH_CASES))
def test_flash_d256_ds_route(device, name, dtype):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    B, Lq, Lk, Hq, Hkv, causal, lengths, q_valid, kv_valid = FLASH_CASES[name]
    D, E = 256, FMT[dtype]
    print(f"ds route flash {name} {dtype}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} causal={causal} "
          f"lengths={lengths} q_valid={q_valid} kv_valid={kv_valid}", flush=True)
    q, k, v, do = (_round(x, dtype) for x in rng_normal(90 + len(name), (B, Lq, Hq, D), (B, Lk, Hkv, D),
                                                        (B, Lk, Hkv, D), (B, Lq, Hq, D)))
    scale = 1.0 / math.sqrt(D)
    mask = _omask(causal, lengths, q_valid, kv_valid, Lq, Lk)
    o, lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, dtype=dtype, return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, sm_scale=scale, dtype=dtype)
    tdt = _tdt(dtype)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    args = [to_dev(x, device, tdt) for x in (q, k, v, o, do)] + [torch.from_numpy(lse).to(device)]
    kw = dict(sm_scale=scale, causal=causal, kv_lengths=L, q_valid=q_valid, kv_valid=kv_valid)
    got = flash_attention_bwd(*args, ds_route=True, **kw)
    assert _launched() == [f"wide_bwd_delta_kernel<{E}, 256>", f"wide_bwd_dc_ds_kernel<{E}, 256, 256, false>",
                           f"wide_bwd_dq_ds_kernel<{E}, 256>"], _launched()
    ref = flash_attention_bwd(*args, ds_route=False, **kw)
    assert _launched() == [f"wide_bwd_dq_kernel<{E}, 256, 256, false, 0, 0>",
                           f"wide_bwd_dc_kernel<{E}, 256, 256, false>"], _launched()
    torch.cuda.synchronize()
    for nm, g, r, w in zip(("dq", "dk", "dv"), got, ref, want):
        assert torch.equal(g, r), f"{nm}: the dS route differs from the two-kernel route"
        _check(to_np(g), w, nm)
    if lengths is not None:
        for b, n in enumerate(lengths):
            assert torch.count_nonzero(got[1][b, n:]) == 0 and torch.count_nonzero(got[2][b, n:]) == 0
