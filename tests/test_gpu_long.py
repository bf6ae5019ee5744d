"""Long sequences: K / V / latent tensors past 2^31 bytes, so every byte
offset into them needs more than 32 bits, in the flash, split-KV and latent
kernels' address arithmetic.

The oracle cannot run these sizes in a test's time, so each case checks a
subset of rows (the last query tile, which sees every key, and a few early
ones) against a plain PyTorch float32 computation on the device from the same
16-bit inputs (P rounded to the input dtype before P.V, as the kernels and
attention_xla.py:349 do), within the 16-bit bar of 2e-2 max-abs.
"""

import math

import pytest

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _ref_rows(q, k, v, rows, scale, causal, kv_len=None):
    """fp32 attention of the query rows ``rows`` of one (batch, head) slice:
    q [Lq, D], k/v [Lk, D] (16-bit) -> [len(rows), Dv]."""
    import torch

    qs = q[rows].float()
    s = (qs @ k.float().T) * scale
    lk = k.shape[0]
    keep = torch.ones_like(s, dtype=torch.bool)
    if kv_len is not None:
        keep &= torch.arange(lk, device=s.device)[None, :] < kv_len
    if causal:
        keep &= torch.arange(lk, device=s.device)[None, :] <= torch.as_tensor(rows, device=s.device)[:, None]
    s = s.masked_fill(~keep, float("-inf"))
    m = s.max(dim=1, keepdim=True).values
    p = torch.exp(s - m)
    l = p.sum(dim=1, keepdim=True)
    return (p.to(v.dtype).float() @ v.float()) / l


def test_flash_forward_4m_keys(device):
    """256 queries over 4 Mi keys (K and V 2 GiB each, B=1, H=2, D=128),
    non-causal with a KV length, and the causal form (queries aligned at key
    0): fp32 rows of the first and last query tiles."""
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    Lq, Lk, H, D = 256, 1 << 22, 2, 128
    print(f"flash fwd long Lq={Lq} Lk={Lk} H={H} D={D}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(71)
    q = torch.randn((1, Lq, H, D), generator=g, device=device).to(torch.bfloat16)
    k, v = (torch.randn((1, Lk, H, D), generator=g, device=device).to(torch.bfloat16) for _ in range(2))
    scale = 1 / math.sqrt(D)
    n = Lk - 12345
    out = flash_attention_fwd(q, k, v, sm_scale=scale, kv_lengths=torch.tensor([n], dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    rows = [0, 1, 100, 127, 128, 255]
    for h in range(H):
        want = _ref_rows(q[0, :, h], k[0, :, h], v[0, :, h], rows, scale, False, kv_len=n)
        err = (out[0, rows, h].float() - want).abs().max().item()
        print(f"  head {h}: max-abs {err:.3e}", flush=True)
        assert err <= TOL
    out = flash_attention_fwd(q, k, v, sm_scale=scale, causal=True)
    torch.cuda.synchronize()
    for h in range(H):
        want = _ref_rows(q[0, :, h], k[0, :, h], v[0, :, h], rows, scale, True)
        err = (out[0, rows, h].float() - want).abs().max().item()
        assert err <= TOL, f"causal head {h}: {err:.3e}"


def test_splitkv_decode_1m(device):
    """Split-KV decode over a 2^20-key cache (K and V 2 GiB each: B=4, Hkv=2,
    D=128), both load paths, lengths full, partial, tiny and full."""
    import torch
    from probjax_amd.hip_attention import splitkv_decode

    B, S, Hq, Hkv, D = 4, 1 << 20, 8, 2, 128
    lens = [S, 600001, 3, S]
    print(f"decode long B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} lengths={lens}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(72)
    q = torch.randn((B, 1, Hq, D), generator=g, device=device).to(torch.bfloat16)
    k, v = (torch.randn((B, S, Hkv, D), generator=g, device=device).to(torch.bfloat16) for _ in range(2))
    L = torch.tensor(lens, dtype=torch.int32, device=device)
    scale = 1 / math.sqrt(D)
    for stream in ("0", "1"):
        import os

        os.environ["PJX_DECODE_STREAM"] = stream
        try:
            out = splitkv_decode(q, k, v, sm_scale=scale, kv_lengths=L)
        finally:
            del os.environ["PJX_DECODE_STREAM"]
        torch.cuda.synchronize()
        for b in range(B):
            for h in range(Hq):
                kv = h // (Hq // Hkv)
                want = _ref_rows(q[b, :, h], k[b, :, kv], v[b, :, kv], [0], scale, False, kv_len=lens[b])
                err = (out[b, 0, h].float() - want[0]).abs().max().item()
                assert err <= TOL, f"stream={stream} b={b} h={h}: {err:.3e}"
        print(f"  stream={stream} ok", flush=True)


def test_latent_decode_2m(device):
    """Latent decode over 2^21 cached rows of rank 576 (2.25 GiB per
    sequence), 16 folded heads, one full and one partial sequence."""
    import torch
    from probjax_amd.hip_attention import mla_decode

    B, S, H, R, DV = 2, 1 << 21, 16, 576, 512
    lens = [S, 1234567]
    print(f"latent decode long B={B} S={S} H={H} R={R}", flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(73)
    q = torch.randn((B, 1, H, R), generator=g, device=device).to(torch.bfloat16)
    cache = torch.randn((B, S, R), generator=g, device=device).to(torch.bfloat16)
    L = torch.tensor(lens, dtype=torch.int32, device=device)
    scale = 1 / math.sqrt(192)
    out = mla_decode(q, cache, sm_scale=scale, v_dim=DV, kv_lengths=L)
    torch.cuda.synchronize()
    for b in range(B):
        want = _ref_rows(q[b, 0], cache[b], cache[b, :, :DV], list(range(H)), scale, False, kv_len=lens[b])
        err = (out[b, 0].float() - want).abs().max().item()
        print(f"  b={b}: max-abs {err:.3e}", flush=True)
        assert err <= TOL
