"""Zero-length inputs through every entry point.

The reference's CPU path gives a row without a valid key output 0 and LSE
+inf (``l == 0``, attention_xla.py:339-429), and empty arrays for Lq = 0 or
B = 0.  Here a key axis of length 0 (torch hands such tensors to the C-ABI as
null pointers) gives exactly that through the flash forward, both decodes
and the latent forward; gradients with no key (dq) or no query (dk, dv,
dcache) are exact zeros; B = 0 and Lq = 0 return empty results.  The
wrappers allocate their outputs uninitialised, so a result the library does
not write fails the exact-zero checks with whatever the memory held.
"""

import math

import pytest

pytestmark = pytest.mark.gpu

DTYPES = ["bf16", "f16", "f32"]


def _dt(name):
    import torch

    return {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[name]


def _randn(shape, dtype, device, seed=0):
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g).to(device=device, dtype=dtype)


def _assert_keyless(o, lse):
    import torch

    assert torch.equal(o, torch.zeros_like(o))
    if lse is not None:
        assert bool(torch.isposinf(lse).all())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_forward_without_keys(device, dtype, D, causal):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    dt = _dt(dtype)
    B, Lq, H = 2, 37, 4
    q = _randn((B, Lq, H, D), dt, device)
    k = torch.empty((B, 0, H, D), dtype=dt, device=device)
    print(f"flash fwd no keys: {dtype} D={D} causal={causal}", flush=True)
    o, lse = flash_attention_fwd(q, k, k, sm_scale=1 / math.sqrt(D), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert o.shape == q.shape and lse.shape == (B, H, Lq)
    _assert_keyless(o, lse)


def test_flash_forward_empty_queries_and_batch(device):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    dt = torch.bfloat16
    k = _randn((2, 50, 4, 128), dt, device)
    o = flash_attention_fwd(torch.empty((2, 0, 4, 128), dtype=dt, device=device), k, k, sm_scale=0.1)
    assert o.shape == (2, 0, 4, 128)
    e = torch.empty((0, 10, 4, 128), dtype=dt, device=device)
    o2, lse2 = flash_attention_fwd(e, e, e, sm_scale=0.1, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert o2.shape == (0, 10, 4, 128) and lse2.shape == (0, 4, 10)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("D", [64, 128, 256])
def test_flash_backward_without_keys_or_queries(device, dtype, D):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    dt = _dt(dtype)
    B, L, H = 2, 45, 4
    print(f"flash bwd empty sides: {dtype} D={D}", flush=True)
    # no keys: dq = 0, dk / dv empty
    q = _randn((B, L, H, D), dt, device, 1)
    k = torch.empty((B, 0, H, D), dtype=dt, device=device)
    o = torch.zeros_like(q)
    do = _randn((B, L, H, D), dt, device, 2)
    lse = torch.full((B, H, L), float("inf"), device=device)
    dq, dk, dv = flash_attention_bwd(q, k, k, o, do, lse, sm_scale=0.1)
    torch.cuda.synchronize()
    assert dk.shape == k.shape and dv.shape == k.shape
    assert torch.equal(dq, torch.zeros_like(dq))
    # no queries: dk = dv = 0, dq empty
    q0 = torch.empty((B, 0, H, D), dtype=dt, device=device)
    kk = _randn((B, L, H, D), dt, device, 3)
    lse0 = torch.empty((B, H, 0), device=device)
    dq0, dk0, dv0 = flash_attention_bwd(q0, kk, kk, q0, q0, lse0, sm_scale=0.1, causal=True)
    torch.cuda.synchronize()
    assert dq0.shape == q0.shape
    assert torch.equal(dk0, torch.zeros_like(dk0)) and torch.equal(dv0, torch.zeros_like(dv0))


@pytest.mark.parametrize("dtype", DTYPES)
def test_splitkv_decode_without_keys(device, dtype):
    import torch
    from probjax_amd.hip_attention import splitkv_decode

    dt = _dt(dtype)
    q = _randn((3, 1, 8, 128), dt, device)
    k = torch.empty((3, 0, 2, 128), dtype=dt, device=device)
    o, lse = splitkv_decode(q, k, k, sm_scale=0.1, return_lse=True)
    torch.cuda.synchronize()
    assert o.shape == q.shape
    _assert_keyless(o, lse)


def test_latent_paths_without_keys_or_queries(device):
    import torch
    from probjax_amd.hip_attention import mla_bwd, mla_decode, mla_fwd

    dt = torch.bfloat16
    B, L, H, R, dv = 2, 40, 4, 576, 512
    q = _randn((B, L, H, R), dt, device)
    c0 = torch.empty((B, 0, R), dtype=dt, device=device)
    # prefill over an empty cache: output 0, LSE +inf
    o, lse = mla_fwd(q, c0, sm_scale=0.07, v_dim=dv, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert o.shape == (B, L, H, dv)
    _assert_keyless(o, lse)
    # decode over an empty cache
    od, lsed = mla_decode(q[:, :1], c0, sm_scale=0.07, v_dim=dv, return_lse=True)
    torch.cuda.synchronize()
    _assert_keyless(od, lsed)
    # backward: no keys -> dq = 0; no queries -> dcache = 0
    do = _randn((B, L, H, dv), dt, device, 4)
    dq, dc = mla_bwd(q, c0, o, do, lse, sm_scale=0.07, causal=True)
    torch.cuda.synchronize()
    assert dc.shape == c0.shape and torch.equal(dq, torch.zeros_like(dq))
    c = _randn((B, 70, R), dt, device, 5)
    q0 = torch.empty((B, 0, H, R), dtype=dt, device=device)
    o0 = torch.empty((B, 0, H, dv), dtype=dt, device=device)
    dq0, dc0 = mla_bwd(q0, c, o0, o0, torch.empty((B, H, 0), device=device), sm_scale=0.07)
    torch.cuda.synchronize()
    assert dq0.shape == q0.shape and torch.equal(dc0, torch.zeros_like(dc0))


def test_public_api_without_keys(device):
    """flex_attention over a zero-length key axis: every row has no valid key,
    so the output is 0 (the l == 0 rule) and no gradient reaches q."""
    import torch
    from probjax_amd import attention as A

    dt = torch.bfloat16
    q = _randn((2, 33, 4, 64), dt, device).requires_grad_(True)
    k = torch.empty((2, 0, 4, 64), dtype=dt, device=device, requires_grad=True)
    out = A.flex_attention(q, k, k)
    assert out.shape == q.shape and torch.equal(out, torch.zeros_like(out))
    out.float().sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(q.grad, torch.zeros_like(q.grad))
