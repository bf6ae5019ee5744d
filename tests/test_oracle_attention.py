"""Pinning of the attention oracle (numpy restatement of xla_attention).

Each check is independent of the restatement's own formula:
* float64 brute force over every (b, h, q) row on tiny inputs;
* torch ``scaled_dot_product_attention`` (CPU, float64) with ``is_causal``,
  boolean ``attn_mask``, additive float mask and ``enable_gqa``;
* invariants from the reference's tests: GQA == ``np.repeat`` K/V
  (probjax tests/test_attention_xla.py:379-405), fully masked rows exactly 0
  (:241-258), bf16 within 2e-2 of fp32 (:408-421), every strategy / tile size
  equal, the natural-log LSE against ``scipy.special.logsumexp``
  (tests/test_attention_gqa_splitkv.py:190-201);
* masked keys contribute exactly nothing (perturbing them leaves the output
  bitwise unchanged) and KVLenMask(L) == a -inf additive bias past L.
"""

import math

import numpy as np
import pytest
import torch
from scipy.special import logsumexp

import oracle
from tests._helpers import rng_normal


def _sdpa(q, k, v, *, scale, causal=False, attn_mask=None):
    t = lambda x: torch.from_numpy(np.asarray(x, np.float64)).transpose(1, 2)  # noqa: E731
    o = torch.nn.functional.scaled_dot_product_attention(
        t(q), t(k), t(v), attn_mask=attn_mask, is_causal=causal, scale=scale,
        enable_gqa=q.shape[2] != k.shape[2],
    )
    return o.transpose(1, 2).numpy()


def _brute(q, k, v, keep, bias, scale):
    """Row-by-row float64 softmax attention; rows without a valid key -> 0."""
    B, Lq, Hq, D = q.shape
    G = Hq // k.shape[2]
    out = np.zeros((B, Lq, Hq, v.shape[-1]))
    for b in range(B):
        for h in range(Hq):
            for i in range(Lq):
                s = np.array([float(np.dot(q[b, i, h].astype(np.float64), k[b, j, h // G]))
                              for j in range(k.shape[1])]) * scale
                if bias is not None:
                    s = s + bias[b if bias.shape[0] > 1 else 0, h if bias.shape[1] > 1 else 0, i]
                ok = keep[b, i]
                if not ok.any():
                    continue
                w = np.exp(s[ok] - s[ok].max())
                out[b, i, h] = (w / w.sum()) @ v[b, ok, h // G].astype(np.float64)
    return out


@pytest.mark.parametrize("strategy", ["dense", "tiled"])
def test_brute_force_tiny_causal_kvlen_bias(strategy):
    B, L, Hq, Hkv, D = 2, 7, 4, 2, 5
    q, k, v, bias = rng_normal(0, (B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D), (B, Hq, L, L))
    lengths = np.array([7, 3], np.int32)
    mask = oracle.CausalMask() & oracle.KVLenMask(lengths)
    keep = np.stack([np.tril(np.ones((L, L), bool)) & (np.arange(L)[None] < n) for n in lengths])
    want = _brute(q, k, v, keep, bias, 0.3)
    got = oracle.xla_attention(q, k, v, mask=mask, bias=oracle.DenseBias(bias), sm_scale=0.3,
                               strategy=strategy, block_q=3, block_k=2)
    np.testing.assert_allclose(got, want, atol=2e-6)


@pytest.mark.parametrize("lq,lk,causal", [(64, 64, True), (300, 300, True), (50, 700, False),
                                          (600, 600, True)])
def test_matches_torch_sdpa(lq, lk, causal):
    q, k, v = rng_normal(1, (2, lq, 4, 32), (2, lk, 4, 32), (2, lk, 4, 32))
    want = _sdpa(q, k, v, scale=0.17, causal=causal)
    got = oracle.xla_attention(q, k, v, mask=oracle.CausalMask() if causal else None, sm_scale=0.17)
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_gqa_kvlen_matches_torch_and_repeat():
    q, k, v = rng_normal(2, (2, 5, 8, 16), (2, 300, 2, 16), (2, 300, 2, 16))
    lengths = np.array([300, 41], np.int32)
    m = torch.from_numpy(np.arange(300)[None, :] < lengths[:, None])[:, None, None, :]
    want = _sdpa(q, k, v, scale=0.25, attn_mask=m)
    got = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=0.25)
    np.testing.assert_allclose(got, want, atol=2e-6)
    rep = oracle.xla_attention(q, np.repeat(k, 4, axis=2), np.repeat(v, 4, axis=2),
                               mask=oracle.KVLenMask(lengths), sm_scale=0.25)
    np.testing.assert_allclose(got, rep, atol=1e-6)


def test_dense_bias_matches_torch_float_mask():
    q, k, v, bias = rng_normal(3, (1, 40, 2, 16), (1, 40, 2, 16), (1, 40, 2, 16), (1, 2, 40, 40))
    want = _sdpa(q, k, v, scale=0.25, attn_mask=torch.from_numpy(bias.astype(np.float64)))
    got = oracle.xla_attention(q, k, v, bias=oracle.DenseBias(bias), sm_scale=0.25)
    np.testing.assert_allclose(got, want, atol=2e-6)


def test_kvlen_equals_minus_inf_bias():
    q, k, v = rng_normal(4, (2, 20, 2, 8), (2, 30, 2, 8), (2, 30, 2, 8))
    lengths = np.array([30, 11], np.int32)
    add = np.where(np.arange(30)[None, :] < lengths[:, None], 0.0, -np.inf).astype(np.float32)
    add = np.broadcast_to(add[:, None, None, :], (2, 1, 20, 30))
    a = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=0.3)
    b = oracle.xla_attention(q, k, v, bias=oracle.DenseBias(np.ascontiguousarray(add)), sm_scale=0.3)
    np.testing.assert_allclose(a, b, atol=1e-6)


@pytest.mark.parametrize("strategy", ["dense", "tiled"])
def test_fully_masked_rows_zero_and_masked_keys_exact(strategy):
    q, k, v = rng_normal(5, (2, 32, 2, 16), (2, 32, 2, 16), (2, 32, 2, 16))
    mask = oracle.KVLenMask(np.array([0, 20], np.int32))
    o1, lse = oracle.xla_attention(q, k, v, mask=mask, sm_scale=0.25, strategy=strategy,
                                   block_q=8, block_k=8, return_lse=True)
    assert np.all(o1[0] == 0) and np.all(np.isfinite(o1))
    assert np.all(np.isinf(lse[0])) and np.all(lse[0] > 0)
    k2, v2 = k.copy(), v.copy()
    k2[1, 20:] = 1e3
    v2[1, 20:] = -7.0
    o2 = oracle.xla_attention(q, k2, v2, mask=mask, sm_scale=0.25, strategy=strategy,
                              block_q=8, block_k=8)
    np.testing.assert_array_equal(o1, o2)


def test_causal_row0_is_v0():
    q, k, v = rng_normal(6, (1, 16, 2, 8), (1, 16, 2, 8), (1, 16, 2, 8))
    o = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1.0)
    np.testing.assert_allclose(o[:, 0], v[:, 0], atol=1e-7)


def test_constant_scores_average_valid_values():
    """q = 0 gives uniform weights: the output is the mean of the valid values."""
    k, v = rng_normal(7, (1, 10, 1, 4), (1, 10, 1, 4))
    q = np.zeros((1, 3, 1, 4), np.float32)
    o = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask([6]), sm_scale=1.0)
    np.testing.assert_allclose(o[0, :, 0], np.broadcast_to(v[0, :6, 0].mean(0), (3, 4)), atol=1e-6)


@pytest.mark.parametrize("bq,bk", [(16, 16), (64, 32), (100, 7), (128, 128)])
def test_strategies_and_tiles_agree(bq, bk):
    q, k, v = rng_normal(8, (1, 128, 2, 16), (1, 128, 2, 16), (1, 128, 2, 16))
    dense = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=0.2, strategy="dense")
    tiled = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=0.2, strategy="tiled",
                                 block_q=bq, block_k=bk)
    np.testing.assert_allclose(tiled, dense, atol=1e-6)


def test_lse_matches_scipy_logsumexp():
    q, k, v = rng_normal(9, (1, 40, 4, 16), (1, 70, 2, 16), (1, 70, 2, 16))
    _, lse = oracle.xla_attention(q, k, v, sm_scale=0.25, return_lse=True, strategy="tiled",
                                  block_q=16, block_k=16)
    kr = np.repeat(k, 2, axis=2).astype(np.float64)
    s = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kr) * 0.25
    np.testing.assert_allclose(lse, logsumexp(s, axis=-1), atol=1e-5)


def test_bf16_close_to_f32():
    q, k, v = rng_normal(10, (1, 64, 2, 32), (1, 64, 2, 32), (1, 64, 2, 32))
    ref = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(32))
    for strategy in ("dense", "tiled"):
        out = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(32),
                                   dtype="bf16", strategy=strategy, block_q=16, block_k=16)
        np.testing.assert_array_equal(out, oracle.round_bf16(out))  # output is bf16-valued
        assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 2e-2


def test_bf16_rounds_p_before_pv():
    """With bf16 inputs, P is rounded to bf16 before P.V (attention_xla.py:349).

    A planted change (no rounding of P) moves the output by more than the
    bf16 output rounding for this input, so the check can fail."""
    q = np.zeros((1, 1, 1, 4), np.float32)
    k = np.zeros((1, 3, 1, 4), np.float32)
    v = np.zeros((1, 3, 1, 4), np.float32)
    q[0, 0, 0, 0] = 1.0
    k[0, 1, 0, 0] = np.log(3.0)  # weights ~1 : 3 : 1 -> P ~ 0.2, 0.6, 0.2 (not bf16-exact)
    v[0, :, 0, 0] = [1.0, -1.0, 1.0]  # output = p0 - p1 + p2 ~ -0.2
    out = oracle.xla_attention(q, k, v, sm_scale=1.0, dtype="bf16", compute_dtype=np.float64)
    s1 = float(oracle.round_bf16(np.array([np.log(3.0)], np.float32))[0])
    p = np.exp(np.array([0.0, s1, 0.0]) - s1)
    p = p / p.sum()
    rp = oracle.round_bf16(p.astype(np.float32)).astype(np.float64)
    want = oracle.round_bf16(np.array([rp[0] - rp[1] + rp[2]], np.float32))[0]
    unrounded = oracle.round_bf16(np.array([p[0] - p[1] + p[2]], np.float32))[0]
    assert want != unrounded  # the check can tell the two apart
    assert out[0, 0, 0, 0] == want


def test_f16_close_to_f32_and_rounds_p():
    """fp16 mode (the reference's fused paths take float16, layers/attention.py:
    1187): fp16-valued output within 2e-3 of fp32 (11 significant bits against
    bf16's 8), and P rounded to fp16 before P.V -- the planted case above,
    where the fp16 rounding of P moves the output by more than its own
    output rounding."""
    q, k, v = rng_normal(10, (1, 64, 2, 32), (1, 64, 2, 32), (1, 64, 2, 32))
    q, k, v = (oracle.round_f16(x) for x in (q, k, v))
    ref = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(32))
    for strategy in ("dense", "tiled"):
        out = oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(32),
                                   dtype="f16", strategy=strategy, block_q=16, block_k=16)
        np.testing.assert_array_equal(out, oracle.round_f16(out))
        assert 0 < np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 2e-3
    q = np.zeros((1, 1, 1, 4), np.float32)
    k = np.zeros((1, 3, 1, 4), np.float32)
    v = np.zeros((1, 3, 1, 4), np.float32)
    q[0, 0, 0, 0] = 1.0
    k[0, 1, 0, 0] = 0.7
    v[0, :, 0, 0] = [1.0, -1.0, 1.0]
    out = oracle.xla_attention(q, k, v, sm_scale=1.0, dtype="f16", compute_dtype=np.float64)
    s1 = float(oracle.round_f16(np.array([0.7], np.float32))[0])
    p = np.exp(np.array([0.0, s1, 0.0]) - s1)
    p = p / p.sum()
    rp = oracle.round_f16(p.astype(np.float32)).astype(np.float64)
    want = oracle.round_f16(np.array([rp[0] - rp[1] + rp[2]], np.float32))[0]
    unrounded = oracle.round_f16(np.array([p[0] - p[1] + p[2]], np.float32))[0]
    assert want != unrounded
    assert out[0, 0, 0, 0] == want


def test_auto_strategy_table():
    assert oracle.auto_strategy(256, 256) == ("dense", None, None)
    assert oracle.auto_strategy(1, 8192)[0] == "dense"
    assert oracle.auto_strategy(512, 512) == ("tiled", 512, 512)
    assert oracle.auto_strategy(4096, 4096) == ("tiled", 256, 256)
