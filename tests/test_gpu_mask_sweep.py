"""Seeded random compositions of probjax's mask and bias classes through
``mha`` on the GPU (forward and dq / dk / dv by autograd), against the oracle's
restatement of the same classes.

Each case draws, from a fixed generator, one or two masks (combined with AND,
sometimes OR or NOT, which lower to a dense mask; at most one of them carries
a payload, as the reference requires), zero to two biases (summed: two
distance terms or two dense terms put all but the first into the dense
bias), a dtype, a head dim, GQA and ragged lengths.  Bars: bf16 / fp16
output max-abs <= 2e-2 against the oracle in the same 16-bit mode, gradients
within probjax's tolerance (tests/test_attention.py:597-626: atol 2e-2,
rtol 1e-2) with atol scaled by max(1, max|ref| / 4); fp32 output <= 1e-5 and
gradients <= 1e-5 * max(1, max|ref|) against float64.  Every case prints its
parameters before it runs.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

MASKS = ("causal", "bottom_right", "window", "causal_window", "kvlen", "qkvlen", "prefix", "seqlen", "segments",
         "block_causal", "key_padding")
STATEFUL = ("kvlen", "prefix", "seqlen", "segments", "block_causal", "key_padding")
BIASES = ("alibi_causal", "alibi_sym", "const", "decay", "softcap", "headscale", "dense")


def _draw(n, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        dt = str(rng.choice(["bf16", "f16", "f32"]))
        d = int(rng.choice([64, 128, 256]))
        b = int(rng.integers(1, 3))
        hkv = int(rng.choice([1, 2]))
        hq = hkv * int(rng.choice([1, 2]))
        lq, lk = int(rng.integers(16, 420)), int(rng.integers(16, 520))
        if b * hq * lq * lk * d > 6e7:
            continue
        masks = [str(m) for m in rng.choice(MASKS, size=int(rng.integers(0, 3)), replace=False)]
        if sum(m in STATEFUL for m in masks) > 1:
            masks = masks[:1]   # the reference refuses to compose two stateful masks (ValueError)
        op = str(rng.choice(["and", "and", "and", "or", "not"])) if masks else "and"
        biases = [str(x) for x in rng.choice(BIASES, size=int(rng.integers(0, 3)), replace=False)]
        if "softcap" in biases and len(biases) > 1:
            biases.remove("softcap")   # a score modifier, not an additive term: keep it alone
        if "headscale" in biases and len(biases) > 1:
            biases.remove("headscale")
        out.append((dt, b, lq, lk, hq, hkv, d, tuple(masks), op, tuple(biases), int(rng.integers(1 << 30))))
    return out


def _build(names, op, biases, b, lq, lk, hq, seed, dev):
    """(API mask, API bias, oracle mask, oracle bias)."""
    import torch
    from probjax_amd import masks as M

    rng = np.random.default_rng(seed)
    am, om = [], []
    for n in names:
        if n == "causal":
            a, o = M.CausalMask(), oracle.CausalMask()
        elif n == "bottom_right":
            a, o = M.CausalFromBottomRightMask(lq, lk), oracle.CausalFromBottomRightMask(lq, lk)
        elif n == "window":
            left, right = int(rng.integers(0, 150)), int(rng.integers(0, 60))
            a, o = M.LocalWindowMask(left, right), oracle.LocalWindowMask(left, right)
        elif n == "causal_window":
            wdw = int(rng.integers(1, 200))
            a, o = M.CausalLocalWindowMask(wdw), oracle.CausalLocalWindowMask(wdw)
        elif n == "kvlen":
            lens = rng.integers(0, lk + 3, size=b).astype(np.int32)
            a, o = M.KVLenMask(torch.from_numpy(lens).to(dev)), oracle.KVLenMask(lens)
        elif n == "qkvlen":
            qv, kv = int(rng.integers(1, lq + 1)), int(rng.integers(1, lk + 1))
            a, o = M.QKVLengthMask(qv, kv), oracle.QKVLengthMask(qv, kv)
        elif n == "prefix":
            p = rng.integers(0, lk + 1, size=b).astype(np.int32)
            a, o = M.PrefixLMMask(torch.from_numpy(p).to(dev)), oracle.PrefixLMMask(p)
        elif n == "seqlen":
            lens = rng.integers(0, min(lq, lk) + 1, size=b).astype(np.int32)
            a, o = M.SeqLenMask(torch.from_numpy(lens).to(dev)), oracle.SeqLenMask(lens)
        elif n in ("segments", "block_causal"):
            if lq != lk:
                continue   # segment ids index queries and keys alike
            ids = np.sort(rng.integers(0, 5, size=(b, lq)), axis=1).astype(np.int32)
            cls = ("SameSegmentMask", "BlockDiagonalCausalMask")[n == "block_causal"]
            a, o = getattr(M, cls)(torch.from_numpy(ids).to(dev)), getattr(oracle, cls)(ids)
        else:  # key_padding: per-query-row key counts, possibly shorter than Lq
            kl = rng.integers(0, lk + 1, size=int(rng.integers(1, lq + 1))).astype(np.int32)
            a, o = M.KeyPaddingMask(torch.from_numpy(kl).to(dev)), oracle.KeyPaddingMask(kl)
        am.append(a)
        om.append(o)
    mask = omask = None
    if am:
        mask, omask = am[0], om[0]
        for a, o in zip(am[1:], om[1:]):
            if op == "or":
                mask, omask = mask | a, omask | o
            else:
                mask, omask = mask & a, omask & o
        if op == "not":
            mask, omask = ~mask, ~omask
    bias = obias = None
    for n in biases:
        if n == "alibi_causal":
            a, o = M.CausalAlibiBias(), oracle.CausalAlibiBias()
        elif n == "alibi_sym":
            a, o = M.SymmetricAlibiBias(), oracle.SymmetricAlibiBias()
        elif n == "const":
            c = float(rng.normal())
            a, o = M.ConstantBias(c), oracle.ConstantBias(c)
        elif n == "decay":
            r = float(rng.uniform(0.01, 0.2))
            a, o = M.DistanceDecayBias(r), oracle.DistanceDecayBias(r)
        elif n == "softcap":
            cap = float(rng.uniform(1.0, 5.0))
            a, o = M.SoftCappingBias(cap), oracle.SoftCappingBias(cap)
        elif n == "headscale":
            sc = rng.uniform(0.3, 2.5, size=hq).astype(np.float32)
            a, o = M.PerHeadScaleBias(torch.from_numpy(sc)), oracle.PerHeadScaleBias(sc)
        else:
            shp = (int(rng.choice([1, b])), int(rng.choice([1, hq])), lq, lk)
            t = (rng.standard_normal(shp) * 0.5).astype(np.float32)
            a, o = M.DenseBias(torch.from_numpy(t).to(dev)), oracle.DenseBias(t)
        bias, obias = (a, o) if bias is None else (bias + a, obias + o)
    return mask, bias, omask, obias


@pytest.mark.parametrize("dt,b,lq,lk,hq,hkv,d,masks,op,biases,seed", _draw(80, 909))
def test_mask_bias_sweep(device, dt, b, lq, lk, hq, hkv, d, masks, op, biases, seed):
    import torch
    from probjax_amd import attention as A

    print(f"mask sweep {dt} B={b} Lq={lq} Lk={lk} Hq={hq} Hkv={hkv} D={d} masks={masks} op={op} "
          f"biases={biases} seed={seed}", flush=True)
    mask, bias, omask, obias = _build(masks, op, biases, b, lq, lk, hq, seed, device)
    q, k, v, do = rng_normal(seed % 1000, (b, lq, hq, d), (b, lk, hkv, d), (b, lk, hkv, d), (b, lq, hq, d))
    low = dt != "f32"
    if low:
        q, k, v, do = (oracle.round_to(x, dt) for x in (q, k, v, do))
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dt]
    scale = 1.0 / math.sqrt(d)
    tq, tk, tv = (to_dev(x, device, tdt).requires_grad_(True) for x in (q, k, v))
    out = A.mha(tq, tk, tv, mask=mask, bias=bias, sm_scale=scale)
    (out.float() * to_dev(do, device, torch.float32)).sum().backward()
    torch.cuda.synchronize()
    cdt = np.float32 if low else np.float64
    o_want, lse = oracle.xla_attention(q, k, v, mask=omask, bias=obias, sm_scale=scale, strategy="dense",
                                       dtype=dt, compute_dtype=cdt, return_lse=True)
    want = attention_backward(q, k, v, o_want, do, lse, mask=omask, bias=obias, sm_scale=scale, dtype=dt,
                              compute_dtype=cdt)
    err = max_abs(to_np(out), o_want)
    print(f"  output max-abs {err:.3e}", flush=True)
    assert err <= (2e-2 if low else 1e-5)
    for nm, t, w in zip(("dq", "dk", "dv"), (tq, tk, tv), want):
        g = to_np(t.grad).astype(np.float64)
        w = np.asarray(w, np.float64)
        e = np.abs(g - w)
        if low:
            atol = 2e-2 * max(1.0, float(np.max(np.abs(w))) / 4.0)
            assert (e <= atol + 1e-2 * np.abs(w)).all(), f"{nm}: max err {e.max():.3e}"
        else:
            assert e.max() <= 1e-5 * max(1.0, float(np.max(np.abs(w)))), f"{nm}: max err {e.max():.3e}"
