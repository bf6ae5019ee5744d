"""float16 end to end on the GPU.

probjax's fused paths take float16 as well as bfloat16 and float32
(layers/attention.py:1187, kernels/attention.py:2678).  Here the 16-bit
kernels run with fp16 operands (v_mfma_f32_*_f16; P and dS rounded to fp16,
fp16 outputs) through ``mha``, ``flex_attention``, ``dot_product_attention``,
the split-KV decode and ``mla``, and are compared with the oracle in fp16 mode
(inputs, P, dS and outputs rounded to fp16 as the reference's casts do,
attention_xla.py:349, 679; attention.py:1042-1056).

Tolerances: outputs max-abs <= 2e-2 against the oracle (the bar of the bf16
tests); gradients within probjax's gradient tolerance (atol 2e-2 scaled by
max(1, max|ref| / 4), rtol 1e-2, tests/test_attention.py:597-626).  Since
both bars would also pass a computation in bf16, every check also requires
the RMS error against the fp16 oracle to be below half the RMS distance
between the oracle's own bf16 and fp16 modes on the same inputs: fp16's 11
significant bits must show.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu


def _rms(a, b):
    d = np.asarray(a, np.float64) - np.asarray(b, np.float64)
    return float(np.sqrt(np.mean(d * d))) if d.size else 0.0


def _check(name, got, want, want_bf16, grad=False):
    """got: kernel result; want: fp16-mode oracle; want_bf16: bf16-mode oracle
    of the same fp16 inputs."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    rms, gap = _rms(got, want), _rms(want_bf16, want)
    print(f"  {name}: max err {err.max() if err.size else 0:.3e}, rms {rms:.3e} "
          f"(bf16-mode oracle at rms {gap:.3e})", flush=True)
    if grad:
        atol = 2e-2 * max(1.0, float(np.max(np.abs(want))) / 4.0)
        assert (err <= atol + 1e-2 * np.abs(want)).all(), f"{name}: max err {err.max():.3e}"
    else:
        assert err.max() <= 2e-2, f"{name}: max err {err.max():.3e}"
    assert rms <= 0.5 * gap, f"{name}: rms {rms:.3e} is not fp16-accurate (bf16 gap {gap:.3e})"


def _masks(kind, B, Lk, device):
    import torch
    from probjax_amd import masks as M

    if kind is None:
        return None, None
    if kind == "causal":
        return M.CausalMask(), oracle.CausalMask()
    if kind == "kvlen":
        lens = np.array([Lk, max(1, Lk // 3)] + [Lk - 5] * (B - 2), np.int32)[:B]
        return M.KVLenMask(torch.from_numpy(lens).to(device)), oracle.KVLenMask(lens)
    if kind == "window":
        return M.LocalWindowMask(64, 32), oracle.LocalWindowMask(64, 32)
    raise AssertionError(kind)


# (name, B, Lq, Lk, Hq, Hkv, D, mask, bias, grad)
CASES = [
    ("causal_d128", 2, 512, 512, 8, 8, 128, "causal", None, True),          # pipelined kernel, 64-key tiles
    ("big_grid_d128", 8, 128, 256, 96, 96, 128, None, None, False),         # pipelined kernel, 32-key tiles
    ("gqa_kvlen_d64", 2, 300, 333, 8, 2, 64, "kvlen", None, True),
    ("bias_ring_d128", 2, 256, 256, 4, 4, 128, None, "dense", True),        # LDS bias ring
    ("bias_regs_d64", 1, 130, 171, 2, 1, 64, "causal", "dense", True),      # bias in registers (Lk % 4 != 0)
    ("window_d64", 1, 300, 300, 4, 2, 64, "window", None, True),            # interval masks
    ("window_alibi_d128", 1, 256, 256, 4, 4, 128, "window", "alibi", True),  # score modifiers
    ("causal_d256", 1, 384, 384, 4, 2, 256, "causal", None, True),          # wide kernels
    ("kvlen_bias_d256", 2, 160, 256, 2, 1, 256, "kvlen", "dense", True),
    ("causal_d192", 1, 256, 256, 2, 2, 192, "causal", None, True),          # zero-padded to 256
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fp16_forward_and_grads(device, case):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    name, B, Lq, Lk, Hq, Hkv, D, mkind, bkind, grad = case
    print(f"fp16 {name}: B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} D={D} mask={mkind} bias={bkind} "
          f"grad={grad}", flush=True)
    seed = 600 + CASES.index(case)
    q, k, v, do = (oracle.round_f16(x) for x in rng_normal(seed, (B, Lq, Hq, D), (B, Lk, Hkv, D),
                                                          (B, Lk, Hkv, D), (B, Lq, Hq, D)))
    mm, om = _masks(mkind, B, Lk, device)
    mb = ob = tb = None
    if bkind == "dense":
        (bias,) = rng_normal(seed + 1, (B, Hq, Lq, Lk), scale=0.5)
        tb = to_dev(bias, device, torch.float32).requires_grad_(grad)
        mb, ob = M.DenseBias(tb), oracle.DenseBias(bias)
    elif bkind == "alibi":
        mb, ob = M.SymmetricAlibiBias(), oracle.SymmetricAlibiBias()
    h = torch.float16
    tq, tk, tv = (to_dev(x, device, h).requires_grad_(grad) for x in (q, k, v))
    if bkind == "dense":  # the route that differentiates the bias data
        out = A.dot_product_attention(tq, tk, tv, mask=mm, bias=mb)
    else:
        out = A.flex_attention(tq, tk, tv, mask=mm, bias=mb, enable_gqa=Hq != Hkv)
    assert out.dtype == h and out.shape == (B, Lq, Hq, D)
    if grad:
        (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()

    scale = 1.0 / math.sqrt(D)
    ref = {}
    for dt in ("f16", "bf16"):
        o, lse = oracle.xla_attention(q, k, v, mask=om, bias=ob, sm_scale=scale, strategy="dense", dtype=dt,
                                      return_lse=True)
        ref[dt] = (o, lse)
    _check("output", to_np(out), ref["f16"][0], ref["bf16"][0])
    if not grad:
        return
    res = {dt: attention_backward(q, k, v, ref[dt][0], do, ref[dt][1], mask=om, bias=ob, sm_scale=scale,
                                  dtype=dt, return_dbias=tb is not None) for dt in ("f16", "bf16")}
    pairs = [("dq", tq), ("dk", tk), ("dv", tv)] + ([("dbias", tb)] if tb is not None else [])
    for i, (nm, t) in enumerate(pairs):
        assert t.grad.dtype == t.dtype
        _check(nm, to_np(t.grad), res["f16"][i], res["bf16"][i], grad=True)


def test_fp16_mha_and_dot_product_attention(device):
    """``mha`` (GQA, causal) and ``dot_product_attention`` with a Flax boolean
    mask array and a bias array take fp16 on the kernels."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    B, L, Hq, Hkv, D = 2, 256, 8, 2, 128
    q, k, v = (oracle.round_f16(x) for x in rng_normal(640, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D)))
    scale = 1.0 / math.sqrt(D)
    h = torch.float16
    got = A.mha(to_dev(q, device, h), to_dev(k, device, h), to_dev(v, device, h), mask=M.CausalMask(),
                sm_scale=scale)
    want = {dt: oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=scale, strategy="dense", dtype=dt)
            for dt in ("f16", "bf16")}
    assert got.dtype == h
    _check("mha", to_np(got), want["f16"], want["bf16"])

    # dot_product_attention: [B, L, H, D] with H = Hkv (no GQA in the Flax API)
    kf, vf = (np.repeat(x, Hq // Hkv, axis=2) for x in (k, v))
    keep = np.tril(np.ones((L, L), bool))
    (bias,) = rng_normal(641, (1, Hq, L, L), scale=0.5)
    tmask = torch.from_numpy(keep)[None, None].to(device)
    got = A.dot_product_attention(to_dev(q, device, h), to_dev(kf, device, h), to_dev(vf, device, h),
                                  mask=tmask, bias=to_dev(bias, device, torch.float32))
    ob = oracle.DenseBias(bias)
    want = {dt: oracle.xla_attention(q, kf, vf, mask=oracle.CausalMask(), bias=ob, sm_scale=scale,
                                     strategy="dense", dtype=dt) for dt in ("f16", "bf16")}
    assert got.dtype == h
    _check("dot_product_attention", to_np(got), want["f16"], want["bf16"])


# (B, Lq, S, Hq, Hkv, D, lengths)
# (the route takes Lq <= 64 with at least 1024 keys, kernels/attention.py:2649-2650)
DECODE = [
    (3, 1, 1100, 8, 2, 128, [1100, 513, 1]),   # 4 rows per KV head
    (2, 4, 1500, 32, 4, 128, [1500, 700]),     # 32 rows: two 16-row blocks
    (2, 8, 1024, 16, 2, 64, None),             # 64 rows: four blocks
]


@pytest.mark.parametrize("B,Lq,S,Hq,Hkv,D,lengths", DECODE)
def test_fp16_splitkv_decode(device, monkeypatch, B, Lq, S, Hq, Hkv, D, lengths):
    import torch
    from probjax_amd import attention as A
    from probjax_amd import hip_attention as H
    from probjax_amd import masks as M

    print(f"fp16 decode B={B} Lq={Lq} S={S} Hq={Hq} Hkv={Hkv} D={D} lengths={lengths}", flush=True)
    q, k, v = (oracle.round_f16(x) for x in rng_normal(650 + Lq, (B, Lq, Hq, D), (B, S, Hkv, D), (B, S, Hkv, D)))
    om = None if lengths is None else oracle.KVLenMask(np.array(lengths, np.int32))
    mm = None if lengths is None else M.KVLenMask(torch.tensor(lengths, dtype=torch.int32, device=device))
    calls = []
    real = H.splitkv_decode
    monkeypatch.setattr(H, "splitkv_decode", lambda *a, **kw: calls.append(1) or real(*a, **kw))
    h = torch.float16
    got = A.flex_attention(*(to_dev(x, device, h) for x in (q, k, v)), mask=mm, enable_gqa=True)
    assert calls, "fp16 decode should run the split-KV kernel"
    assert got.dtype == h
    scale = 1.0 / math.sqrt(D)
    want = {dt: oracle.xla_attention(q, k, v, mask=om, sm_scale=scale, strategy="dense", dtype=dt)
            for dt in ("f16", "bf16")}
    _check("decode", to_np(got), want["f16"], want["bf16"])


def test_fp16_mla_decode_and_latent_prefill(device):
    """Absorbed ``mla`` in fp16: the split-KV latent decode and the latent
    flash forward / backward (rank 576, v_dim 512)."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    h = torch.float16
    scale = 1.0 / math.sqrt(192)
    # decode: 16 heads, one query, ragged lengths
    B, S, H, R, dv = 3, 700, 16, 576, 512
    q, c = (oracle.round_f16(x) for x in rng_normal(660, (B, 1, H, R), (B, S, R)))
    lens = np.array([700, 300, 65], np.int32)
    got = A.mla(to_dev(q, device, h), to_dev(c, device, h), mask=M.KVLenMask(torch.from_numpy(lens).to(device)),
                sm_scale=scale, v_dim=dv)
    shared = c[:, :, None, :]
    want = {dt: oracle.xla_attention(q, shared, shared, mask=oracle.KVLenMask(lens), sm_scale=scale,
                                     strategy="dense", dtype=dt)[..., :dv] for dt in ("f16", "bf16")}
    assert got.dtype == h
    _check("mla decode", to_np(got), want["f16"], want["bf16"])

    # causal prefill with gradients
    B, L, H = 1, 256, 8
    q, c, do = (oracle.round_f16(x) for x in rng_normal(661, (B, L, H, R), (B, L, R), (B, L, H, dv)))
    tq = to_dev(q, device, h).requires_grad_(True)
    tc = to_dev(c, device, h).requires_grad_(True)
    out = A.mla(tq, tc, mask=M.CausalMask(), sm_scale=scale, v_dim=dv)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    shared = c[:, :, None, :]
    dop = np.concatenate([do, np.zeros(do.shape[:-1] + (R - dv,), np.float32)], axis=-1)
    ref = {}
    for dt in ("f16", "bf16"):
        o, lse = oracle.xla_attention(q, shared, shared, mask=oracle.CausalMask(), sm_scale=scale,
                                      strategy="dense", dtype=dt, return_lse=True)
        dq, dk, dvv = attention_backward(q, shared, shared, o, dop, lse, mask=oracle.CausalMask(),
                                         sm_scale=scale, dtype=dt)
        ref[dt] = (o[..., :dv], dq, (np.asarray(dk, np.float64) + np.asarray(dvv, np.float64))[:, :, 0])
    _check("latent output", to_np(out), ref["f16"][0], ref["bf16"][0])
    _check("latent dq", to_np(tq.grad), ref["f16"][1], ref["bf16"][1], grad=True)
    _check("latent dcache", to_np(tc.grad), ref["f16"][2], ref["bf16"][2], grad=True)


def test_fp16_materialized_mla(device):
    """Projected ``mla`` in fp16 (up-projection kernel, then the flash
    kernels) against the oracle's materialised path."""
    import torch
    from probjax_amd import attention as A
    from probjax_amd import masks as M

    B, L, H, R, dk, dv = 2, 160, 4, 96, 64, 48
    q, c, wk, wv = (oracle.round_f16(x) for x in rng_normal(670, (B, L, H, dk), (B, L, R), (H, dk, R), (H, dv, R),
                                                           scale=0.3))
    h = torch.float16
    got = A.mla(*(to_dev(x, device, h) for x in (q, c, wk, wv)), mask=M.CausalMask(), sm_scale=1 / 8)
    assert got.dtype == h and got.shape == (B, L, H, dv)
    want = {dt: oracle.materialized_mla(q, c, wk, wv, mask=oracle.CausalMask(), sm_scale=1 / 8, dtype=dt)
            for dt in ("f16", "bf16")}
    _check("materialised mla", to_np(got), want["f16"], want["bf16"])
    assert max_abs(to_np(got), want["f16"]) <= 2e-2
