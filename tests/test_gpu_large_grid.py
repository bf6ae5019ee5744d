"""Parity of the 16-bit D = 128 forward at large grids with the oracle.

Without bias or extended masks, grids of at least three 128-row query tiles
per CU run ``flash_fwd_bf16_pipe_kernel<E, 128, 32, 3>`` (32-key tiles, three
workgroups per CU); smaller grids run the 64-key form, which the other tests
cover.  Every case here is sized past that threshold (asserted against the
device's CU count): ragged query and key lengths (partial 128-row and 32-key
tiles), GQA, causal with Lq != Lk, per-batch KV lengths including 0 (rows
with no key: output 0, LSE +inf), QKVLengthMask and fp16.

Tolerances: outputs max-abs <= 2e-2 against the fp32 oracle on the same
16-bit inputs (the bar of the other 16-bit tests), LSE max-abs <= 1e-2 where
finite and +inf exactly where the oracle's is; fp16 additionally within half
the RMS distance between the oracle's bf16 and fp16 modes.
"""

import math

import numpy as np
import pytest

import oracle
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _rms(a, b):
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    return float(np.sqrt(np.mean(d * d))) if d.size else 0.0


def _assert_large_grid(B, Lq, Hq):
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks = -(-Lq // 128) * B * Hq
    assert blocks >= 3 * cus, f"{blocks} query tiles of 128 rows do not reach the 32-key kernel ({cus} CUs)"


CASES = {
    # name: B, Lq, Lk, Hq, Hkv, causal, kv_lengths, (q_valid, kv_valid)
    "causal_ragged": (2, 1100, 1100, 48, 48, True, None, None),
    "causal_gqa8": (1, 2000, 2000, 64, 8, True, None, None),
    "noncausal_lq_gt_lk": (1, 1536, 1000, 64, 16, False, None, None),
    "causal_lq_lt_lk": (1, 1536, 2100, 64, 64, True, None, None),
    "causal_kvlen": (4, 1024, 1024, 24, 24, True, [1024, 700, 33, 0], None),
    "noncausal_kvlen_gqa": (2, 1300, 1500, 48, 12, False, [1500, 911], None),
    "qkv_length": (2, 1280, 1280, 40, 40, False, None, (1000, 1100)),
}


@pytest.mark.parametrize("name", list(CASES))
def test_large_grid_bf16_matches_oracle(device, name):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, Lq, Lk, Hq, Hkv, causal, lengths, qkv = CASES[name]
    D = 128
    _assert_large_grid(B, Lq, Hq)
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(11, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D)))
    scale = 1.0 / math.sqrt(D)
    masks = [oracle.CausalMask()] if causal else []
    if lengths is not None:
        masks.append(oracle.KVLenMask(np.array(lengths, np.int32)))
    if qkv is not None:
        masks.append(oracle.QKVLengthMask(*qkv))
    mask = None if not masks else (masks[0] if len(masks) == 1 else oracle.ComposeMask("and", *masks))
    print(f"large grid {name}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} causal={causal} "
          f"lengths={lengths} qkv={qkv}", flush=True)
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=scale, return_lse=True)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    kw = {} if qkv is None else dict(q_valid=qkv[0], kv_valid=qkv[1])
    got, lse = flash_attention_fwd(*(to_dev(x, device, torch.bfloat16) for x in (q, k, v)), sm_scale=scale,
                                   causal=causal, kv_lengths=L, return_lse=True, **kw)
    torch.cuda.synchronize()
    got, lse = to_np(got), to_np(lse)
    err = max_abs(got, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= TOL
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-2
    # rows with no valid key give exactly 0
    dead = np.isposinf(want_lse).transpose(0, 2, 1)  # [B, Lq, Hq]
    assert not np.any(got[dead])


def test_large_grid_fp16_matches_oracle(device):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 1, 1536, 64, 128
    _assert_large_grid(B, L, H)
    q, k, v = (oracle.round_f16(x) for x in rng_normal(12, (B, L, H, D), (B, L, H, D), (B, L, H, D)))
    scale = 1.0 / math.sqrt(D)
    print(f"large grid fp16: B={B} L={L} H={H} causal", flush=True)
    want = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=scale, dtype="f16")
    want_bf16 = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=scale, dtype="bf16")
    got = to_np(flash_attention_fwd(*(to_dev(x, device, torch.float16) for x in (q, k, v)), sm_scale=scale,
                                    causal=True))
    err, rms, gap = max_abs(got, want), _rms(got, want), _rms(want_bf16, want)
    print(f"  max-abs {err:.3e}, rms {rms:.3e} (bf16-mode oracle at rms {gap:.3e})", flush=True)
    assert err <= TOL
    assert rms <= 0.5 * gap


def test_large_grid_deterministic_and_row0_exact(device):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 2, 1536, 32, 128
    _assert_large_grid(B, L, H)
    q, k, v = (to_dev(x, device, torch.bfloat16) for x in rng_normal(13, (B, L, H, D), (B, L, H, D), (B, L, H, D)))
    a = flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True)
    b = flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    # causal row 0 sees key 0 only: its output is v[:, 0] exactly
    assert torch.equal(a[:, 0], v[:, 0])
