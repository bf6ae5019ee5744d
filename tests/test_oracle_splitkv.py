"""Pinning of the split-KV oracle: exact merge, packing, split-count table.

Restates the reference's checks (probjax tests/test_attention_gqa_splitkv.py:
41-53 dense fp32 reference, :170-201 split-KV output + LSE for odd shapes and
split counts) with torch/numpy references instead of the Pallas interpreter.
"""

import math

import numpy as np
import pytest
from scipy.special import logsumexp

import oracle
from oracle.splitkv import merge_partials, pack_queries, split_partials, unpack_rows
from tests._helpers import rng_normal


def _reference(q, k, v, lengths=None):
    """fp32 dense attention with np.repeat GQA semantics (float64)."""
    rep = q.shape[2] // k.shape[2]
    kr, vr = (np.repeat(x.astype(np.float64), rep, axis=2) for x in (k, v))
    s = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kr) / math.sqrt(q.shape[-1])
    if lengths is not None:
        keep = np.arange(k.shape[1])[None, :] < np.asarray(lengths)[:, None]
        s = np.where(keep[:, None, None, :], s, -np.inf)
    lse = logsumexp(s, axis=-1)
    p = np.exp(s - lse[..., None])
    return np.einsum("bhqk,bkhd->bqhd", p, vr), lse


@pytest.mark.parametrize(
    "b,lq,lkv,hq,hkv,d,splits",
    [(1, 1, 200, 4, 4, 16, None), (2, 3, 130, 4, 2, 16, 3), (1, 4, 96, 8, 1, 32, 2),
     (1, 2, 50, 2, 1, 24, 1), (2, 1, 1000, 8, 2, 16, 7)],
)
def test_splitkv_matches_dense(b, lq, lkv, hq, hkv, d, splits):
    q, k, v = rng_normal(lkv, (b, lq, hq, d), (b, lkv, hkv, d), (b, lkv, hkv, d))
    out, lse = oracle.splitkv_forward(q, k, v, sm_scale=1 / math.sqrt(d), num_splits=splits,
                                      block_k=16, return_lse=True)
    want, want_lse = _reference(q, k, v)
    np.testing.assert_allclose(out, want, atol=2e-6)
    np.testing.assert_allclose(lse, want_lse, atol=2e-5)


@pytest.mark.parametrize("split_len", [16, 64, 112, 1024])
def test_merge_is_exact_for_any_split_with_lengths(split_len):
    q, k, v = rng_normal(3, (3, 1, 8, 16), (3, 300, 2, 16), (3, 300, 2, 16))
    lengths = np.array([300, 17, 0], np.int32)
    op, lp = split_partials(q, k, v, sm_scale=0.25, split_len=split_len, kv_lengths=lengths)
    out, lse = merge_partials(op, lp)
    out = unpack_rows(out, 1, 8)
    want = _ref_scaled(q[:2], k[:2], v[:2], lengths[:2], 0.25)
    np.testing.assert_allclose(out[:2], want, atol=2e-6)
    assert np.all(out[2] == 0)  # empty sequence -> zero output
    # every split empty: the reference's base-2 combine gives a huge negative
    # (finite) LSE, unlike the XLA path's +inf
    assert np.all(lse[2] < -1e14)


def _ref_scaled(q, k, v, lengths, scale):
    rep = q.shape[2] // k.shape[2]
    kr, vr = (np.repeat(x.astype(np.float64), rep, axis=2) for x in (k, v))
    s = np.einsum("bqhd,bkhd->bhqk", q.astype(np.float64), kr) * scale
    keep = np.arange(k.shape[1])[None, :] < np.asarray(lengths)[:, None]
    s = np.where(keep[:, None, None, :], s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bhqk,bkhd->bqhd", p, vr)


def test_splitkv_with_lengths_matches_xla_kvlen():
    q, k, v = rng_normal(4, (2, 2, 8, 16), (2, 500, 4, 16), (2, 500, 4, 16))
    lengths = np.array([123, 500], np.int32)
    a = oracle.splitkv_forward(q, k, v, sm_scale=0.3, num_splits=4, kv_lengths=lengths)
    b = oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lengths), sm_scale=0.3)
    np.testing.assert_allclose(a, b, atol=2e-6)


def test_pack_unpack_round_trip_and_row_order():
    (q,) = rng_normal(5, (2, 3, 8, 4))
    p = pack_queries(q, 2)
    assert p.shape == (2, 2, 12, 4)
    # row = g * Lq + t for kv head j: query head j*G + g at position t
    np.testing.assert_array_equal(p[1, 1, 2 * 3 + 1], q[1, 1, 1 * 4 + 2])
    np.testing.assert_array_equal(unpack_rows(p, 3, 8), q)


def test_default_num_splits_table():
    # attention_splitkv.py:106-118: target 2*82 programs, >= 256 keys per split
    assert oracle.default_num_splits(1, 8, 1, 16384, 64) == 21
    assert oracle.default_num_splits(8, 8, 1, 16384, 64) == 3
    assert oracle.default_num_splits(1, 1, 1, 300, 64) == 1
    assert oracle.default_num_splits(32, 8, 1, 8192, 64) == 2
