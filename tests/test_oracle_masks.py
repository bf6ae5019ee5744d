"""Known-answer tests of the oracle's mask/bias objects.

Restates the reference's own known-answer tests for the masks and biases on
the path (probjax tests/test_attention_mask_bias.py:54-68 NoMask/Causal,
:130-136 QKVLengthMask, :152-163 KVLenMask.dense, :191-209 ComposeMask,
:263-294 DenseBias, :425-453 block masks) against closed forms.
"""

import numpy as np
import pytest

import oracle
from oracle.masks import AttentionMask


def _idx(n):
    return np.arange(n, dtype=np.int32)


def _block_from_dense(dense, bq, bk):
    q_len, k_len = dense.shape
    nq, nk = -(-q_len // bq), -(-k_len // bk)
    out = np.zeros((nq, nk), bool)
    for i in range(nq):
        for j in range(nk):
            out[i, j] = dense[i * bq : (i + 1) * bq, j * bk : (j + 1) * bk].any()
    return out


def test_no_mask_all_true():
    m = oracle.NoMask()(_idx(5), _idx(7))
    assert m.shape == (5, 7) and m.all()
    assert oracle.NoMask().block_mask(16, 12, 4, 3) is None


def test_causal_lower_triangular_top_left():
    got = oracle.CausalMask()(_idx(6), _idx(6))
    np.testing.assert_array_equal(got, np.tril(np.ones((6, 6), bool)))
    # top-left aligned also for Q != K: row 0 sees key 0 only
    got = oracle.CausalMask()(_idx(3), _idx(5))
    assert got[0].tolist() == [True, False, False, False, False]


def test_qkv_length_mask_clips_both_axes():
    got = oracle.QKVLengthMask(4, 6)(_idx(7), _idx(9))
    want = (_idx(7)[:, None] < 4) & (_idx(9)[None, :] < 6)
    np.testing.assert_array_equal(got, want)


def test_kv_len_mask_dense():
    lengths = np.array([2, 4, 6], np.int32)
    dense = oracle.KVLenMask(lengths).dense(5, 6, batch_size=3, num_heads=2)
    want = np.broadcast_to((_idx(6)[None, :] < lengths[:, None])[:, None, None, :], (3, 2, 5, 6))
    np.testing.assert_array_equal(dense, want)
    # explicit rows for batch 0: keys 0, 1 valid
    assert dense[0, 1, 3].tolist() == [True, True, False, False, False, False]


def test_kv_len_mask_payload_and_no_block_mask():
    m = oracle.KVLenMask([3, 9])
    data, _ = m.get_data()
    assert data.shape == (2, 1, 1, 1) and data.ravel().tolist() == [3, 9]
    assert m.block_mask(16, 16, 4, 4) is None
    assert m.query_independent and m.stateful


@pytest.mark.parametrize("op", ["and", "or", "xor"])
def test_compose_mask_ops(op):
    a, b = oracle.CausalMask(), oracle.QKVLengthMask(5, 6)
    va, vb = a(_idx(8), _idx(8)), b(_idx(8), _idx(8))
    got = oracle.ComposeMask(op, a, b)(_idx(8), _idx(8))
    want = {"and": va & vb, "or": va | vb, "xor": va ^ vb}[op]
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal((a & b)(_idx(8), _idx(8)), va & vb)


def test_compose_two_stateful_raises():
    with pytest.raises(ValueError, match="Cannot compose two stateful masks"):
        oracle.ComposeMask("and", oracle.KVLenMask([1]), oracle.KVLenMask([2]))


def test_compose_kvlen_and_causal_tile_keep():
    m = oracle.CausalMask() & oracle.KVLenMask([3, 5])
    got = m.tile_keep(1, _idx(6), _idx(6))
    want = np.tril(np.ones((6, 6), bool)) & (_idx(6)[None, :] < 5)
    np.testing.assert_array_equal(got, want)


def test_dense_bias_adds_tile_and_broadcasts():
    scores = np.ones((2, 3), np.float32)
    tile = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = oracle.DenseBias(np.zeros((1, 1, 2, 3), np.float32))
    np.testing.assert_allclose(b(scores, 0, _idx(2), _idx(3), data=tile), scores + tile)
    dense = np.arange(12, dtype=np.float32).reshape(1, 1, 3, 4)
    np.testing.assert_allclose(
        oracle.DenseBias(dense)(np.zeros((3, 4), np.float32), 0, _idx(3), _idx(4)), dense[0, 0]
    )
    got = oracle.DenseBias(dense).dense(3, 4, batch_size=2, num_heads=3)
    np.testing.assert_array_equal(got, np.broadcast_to(dense, (2, 3, 3, 4)))
    with pytest.raises(ValueError, match="requires bias batch dimension to be 1"):
        oracle.DenseBias(np.zeros((2, 1, 3, 4), np.float32))(np.zeros((3, 4)), 0, _idx(3), _idx(4))


def test_dense_bias_tile_add_selects_batch_and_head():
    bias = np.arange(2 * 3 * 4 * 5, dtype=np.float32).reshape(2, 3, 4, 5)
    s = np.zeros((2, 2), np.float32)
    got = oracle.DenseBias(bias).tile_add(s, 1, 2, 2, 2, 3, 2)
    np.testing.assert_array_equal(got, bias[1, 2, 2:4, 3:5])
    # broadcast head: head index ignored
    got = oracle.DenseBias(bias[:, :1]).tile_add(s, 1, 2, 0, 2, 0, 2)
    np.testing.assert_array_equal(got, bias[1, 0, :2, :2])
    # ragged tile is zero padded
    got = oracle.DenseBias(bias).tile_add(np.zeros((3, 3), np.float32), 0, 0, 2, 3, 3, 3)
    assert got[2].tolist() == [0, 0, 0] and got[0, 2] == 0 and got[0, 0] == bias[0, 0, 2, 3]


def test_sum_bias_no_double_counting():
    dense = np.arange(15, dtype=np.float32).reshape(1, 1, 3, 5)
    s = np.full((3, 5), 2.0, np.float32)
    b = oracle.DenseBias(dense) + oracle.DenseBias(dense)
    np.testing.assert_allclose(b.tile_add(s, 0, 0, 0, 3, 0, 5), s + 2 * dense[0, 0])


@pytest.mark.parametrize(
    "mask,q_len,kv_len,bq,bk",
    [
        (oracle.CausalMask(), 11, 10, 4, 3),
        (oracle.QKVLengthMask(6, 7), 9, 11, 4, 3),
        (oracle.CausalMask() & oracle.QKVLengthMask(6, 7), 12, 12, 4, 4),
    ],
)
def test_block_mask_matches_dense_nonempty_blocks(mask, q_len, kv_len, bq, bk):
    dense = mask(_idx(q_len), _idx(kv_len))
    np.testing.assert_array_equal(mask.block_mask(q_len, kv_len, bq, bk), _block_from_dense(dense, bq, bk))
    # the generic (evaluate every tile) fallback agrees
    np.testing.assert_array_equal(AttentionMask.block_mask(mask, q_len, kv_len, bq, bk),
                                  _block_from_dense(dense, bq, bk))


# ---------------------------------------------------------------------------
# Positional / segment masks and score modifiers (restated from the
# reference's tests/test_attention_mask_bias.py:70-173, 296-365).
# ---------------------------------------------------------------------------

def test_local_window_band_and_right_none():
    d = _idx(8)[:, None] - _idx(8)[None, :]
    got = oracle.LocalWindowMask(left_window=2, right_window=1)(_idx(8), _idx(8))
    np.testing.assert_array_equal(got, (d >= -1) & (d <= 2))
    np.testing.assert_array_equal(oracle.LocalWindowMask(3, None)(_idx(8), _idx(8)),
                                  oracle.LocalWindowMask(3, 0)(_idx(8), _idx(8)))


def test_causal_local_window_band():
    d = _idx(8)[:, None] - _idx(8)[None, :]
    got = oracle.CausalLocalWindowMask(left_window=3)(_idx(8), _idx(8))
    np.testing.assert_array_equal(got, (d >= 0) & (d <= 3))


def test_causal_from_bottom_right_alignment():
    got = oracle.CausalFromBottomRightMask(q_length=3, kv_length=5)(_idx(3), _idx(5))
    np.testing.assert_array_equal(got, (_idx(3)[:, None] + 2) >= _idx(5)[None, :])
    # last query row sees every key
    assert got[-1].all() and got[0].sum() == 3


def test_prefix_lm_scalar_and_per_batch():
    got = oracle.PrefixLMMask(np.int32(2))(_idx(6), _idx(6))
    want = (_idx(6)[None, :] < 2) | (_idx(6)[:, None] >= _idx(6)[None, :])
    np.testing.assert_array_equal(got, want)
    m = oracle.PrefixLMMask(np.array([1, 4], np.int32))
    np.testing.assert_array_equal(m.tile_keep(1, _idx(6), _idx(6)),
                                  (_idx(6)[None, :] < 4) | (_idx(6)[:, None] >= _idx(6)[None, :]))
    assert m.block_mask(6, 6, 2, 2) is None


def test_block_diagonal_masks():
    q_ids = np.array([0, 0, 1, 1, 2], np.int32)
    k_ids = np.array([0, 1, 1, 2], np.int32)
    diag = oracle.BlockDiagonalMask(q_ids, k_ids)(_idx(5), _idx(4))
    np.testing.assert_array_equal(diag, q_ids[:, None] == k_ids[None, :])
    causal = oracle.BlockDiagonalCausalMask(q_ids, k_ids)(_idx(5), _idx(4))
    np.testing.assert_array_equal(causal, (q_ids[:, None] == k_ids[None, :])
                                  & (_idx(5)[:, None] >= _idx(4)[None, :]))


def test_seq_len_dense():
    lengths = np.array([2, 4, 6], np.int32)
    m = oracle.SeqLenMask(lengths)
    for b, L in enumerate(lengths):
        valid = _idx(6) < L
        want = (valid[:, None] & valid[None, :]) | np.eye(6, dtype=bool)
        np.testing.assert_array_equal(m.tile_keep(b, _idx(6), _idx(6)), want)


def test_same_segment_ids():
    q_ids = np.array([0, 1, 1, 2], np.int32)
    k_ids = np.array([1, 0, 2, 1, 2], np.int32)
    got = oracle.SameSegmentMask(q_ids, k_ids)(_idx(4), _idx(5))
    np.testing.assert_array_equal(got, q_ids[:, None] == k_ids[None, :])
    # per-batch ids, keys default to the query ids
    ids = np.array([[0, 0, 1, 1], [0, 1, 1, 1]], np.int32)
    m = oracle.SameSegmentMask(ids)
    np.testing.assert_array_equal(m.tile_keep(1, _idx(4), _idx(4)), ids[1][:, None] == ids[1][None, :])


def test_bias_value_formulas():
    scores = np.zeros((4, 4), np.float32)
    h = 1
    slope = 2.0 ** (-(h + 1))
    d = _idx(4)[:, None] - _idx(4)[None, :]
    np.testing.assert_allclose(oracle.CausalAlibiBias()(scores, h, _idx(4), _idx(4)),
                               -slope * np.maximum(d, 0))
    np.testing.assert_allclose(oracle.SymmetricAlibiBias()(scores, h, _idx(4), _idx(4)),
                               -slope * np.abs(d))
    np.testing.assert_allclose(oracle.DistanceDecayBias(alpha=0.7)(scores, h, _idx(4), _idx(4)),
                               -0.7 * np.abs(d), rtol=1e-6)
    np.testing.assert_array_equal(oracle.IdentityBias()(scores, h, _idx(4), _idx(4)), scores)
    np.testing.assert_allclose(oracle.ConstantBias(0.3)(scores, h, _idx(4), _idx(4)), scores + 0.3)


def test_soft_capping_and_grad():
    scores = np.array([[-50.0, 0.0, 50.0]], np.float32)
    b = oracle.SoftCappingBias(softcap=10.0)
    out = b(scores, 0, _idx(1), _idx(3))
    assert np.all(np.abs(out) <= 10.0 + 1e-5)
    np.testing.assert_allclose(out, 10.0 * np.tanh(scores / 10.0))
    g = b.grad(scores)
    assert g.shape == scores.shape and np.all(g >= 0) and np.all(g <= 1)
    # the derivative against central differences
    x = np.linspace(-30, 30, 13).astype(np.float64)[None]
    eps = 1e-5
    num = (b(x + eps, 0, None, None) - b(x - eps, 0, None, None)) / (2 * eps)
    np.testing.assert_allclose(b.grad(x), num, atol=1e-7)
    with pytest.raises(ValueError):
        oracle.SoftCappingBias(0.0)


def test_per_head_scale():
    scores = np.ones((2, 3), np.float32)
    b = oracle.PerHeadScaleBias(np.array([2.0, 0.5], np.float32))
    np.testing.assert_allclose(b(scores, 0, _idx(2), _idx(3)), 2 * scores)
    np.testing.assert_allclose(b(scores, 1, _idx(2), _idx(3)), 0.5 * scores)
    np.testing.assert_allclose(b.grad_tile(scores, 0, 1, 0, 2, 0, 3), 0.5 * scores)


def test_key_padding_known_answer():
    """probjax tests/test_attention_mask_bias.py:182-188: a per-row vector
    payload keeps k < seg_q[q]."""
    seg_q = np.array([1, 3, 5, 6], np.int32)
    got = oracle.KeyPaddingMask(np.array([6], np.int32))(_idx(4), _idx(6), seg_q=seg_q)
    np.testing.assert_array_equal(got, _idx(6)[None, :] < seg_q[:, None])


def test_key_padding_payload_rows():
    """The XLA path reads the payload per query position: a [T] payload is
    shared by every batch ([1, T, 1, 1], attention_mask_bias.py:1186-1187),
    [B, T] is paged by batch, rows past T read the zero fill; a scalar payload
    is KVLenMask with one length."""
    m = oracle.KeyPaddingMask(np.array([16, 12], np.int32))
    for b in range(2):
        keep = m.tile_keep(b, _idx(4), _idx(20))
        np.testing.assert_array_equal(keep[0], _idx(20) < 16)
        np.testing.assert_array_equal(keep[1], _idx(20) < 12)
        assert not keep[2:].any()
    m2 = oracle.KeyPaddingMask(np.array([[3, 1, 2], [0, 5, 5]], np.int32))
    np.testing.assert_array_equal(m2.tile_keep(1, _idx(3), _idx(6)).sum(axis=1), [0, 5, 5])
    np.testing.assert_array_equal(m2.tile_keep(0, _idx(4), _idx(6)).sum(axis=1), [3, 1, 2, 0])
    # a window of rows reads the same counts as the whole
    np.testing.assert_array_equal(m2.tile_keep(0, _idx(4)[1:3], _idx(6)), m2.tile_keep(0, _idx(4), _idx(6))[1:3])
    s = oracle.KeyPaddingMask(np.int32(7))
    kv = oracle.KVLenMask(np.array([7, 7], np.int32))
    for b in range(2):
        np.testing.assert_array_equal(s.tile_keep(b, _idx(5), _idx(9)), kv.tile_keep(b, _idx(5), _idx(9)))
    # boolean payloads compare as 0 / 1
    mb = oracle.KeyPaddingMask(np.array([True, False]))
    np.testing.assert_array_equal(mb.tile_keep(0, _idx(2), _idx(3)).sum(axis=1), [1, 0])


def test_marginalization_and_not_masks():
    """tests/test_attention_mask_bias.py:173-179 (rect plus diagonal) and the
    NotMask / OR / XOR compositions (:191-209); the payload read per query and
    key position in the XLA path, per batch for a [B, T] payload."""
    m = np.array([True, False, True, False])
    got = oracle.MarginalizationMask(m)(_idx(4), _idx(4))
    np.testing.assert_array_equal(got, (m[:, None] & m[None, :]) | np.eye(4, dtype=bool))
    np.testing.assert_array_equal(oracle.MarginalizationMask(m).tile_keep(0, _idx(4), _idx(4)), got)
    mb = np.array([[True, True, False], [False, True, True]])
    for b in range(2):
        want = (mb[b][:, None] & mb[b][None, :]) | np.eye(3, dtype=bool)
        np.testing.assert_array_equal(oracle.MarginalizationMask(mb).tile_keep(b, _idx(3), _idx(3)), want)
    # positions past the payload read the zero fill: only the diagonal survives
    tail = oracle.MarginalizationMask(np.array([True, True])).tile_keep(0, _idx(4), _idx(4))
    np.testing.assert_array_equal(tail[2:], np.eye(4, dtype=bool)[2:])
    c = oracle.CausalMask()
    np.testing.assert_array_equal((~c).tile_keep(0, _idx(5), _idx(5)), ~np.tril(np.ones((5, 5), bool)))
    w = oracle.LocalWindowMask(1, 0)
    got = (c | w).tile_keep(0, _idx(5), _idx(6)) ^ (c ^ w).tile_keep(0, _idx(5), _idx(6))
    np.testing.assert_array_equal(got, (c & w).tile_keep(0, _idx(5), _idx(6)))


def test_relative_position_buckets():
    """T5 bucketing (attention_mask_bias.py:2417-2449) against hand-computed
    values: 16 bidirectional buckets, max_distance 8 -> 8 per direction,
    exact below 4, then 4 + floor(log(rp/4) / log(2) * 4) capped at 7; keys
    after the query (k > q) in the upper half."""
    rel_k_minus_q = np.array([0, -1, -3, -4, -5, -6, -7, -8, -50, 1, 3, 5, 100])
    want = np.array([0, 1, 3, 4, 5, 6, 7, 7, 7, 9, 11, 13, 15])
    got = oracle.masks.relative_position_bucket(rel_k_minus_q, num_buckets=16, max_distance=8, bidirectional=True)
    np.testing.assert_array_equal(got, want)
    # unidirectional: keys after the query share bucket 0
    got = oracle.masks.relative_position_bucket(np.array([2, 0, -2, -9]), num_buckets=8, max_distance=16,
                                                bidirectional=False)
    # (k - q = -9: rp 9 >= 4 exact buckets, 4 + floor(log(9/4) / log(16/4) * 4) = 6)
    np.testing.assert_array_equal(got, [0, 0, 2, 6])


def test_relative_position_biases():
    """tests/test_attention_mask_bias.py:323-350: the T5 table per head, and
    the learned clipped-distance table."""
    table = np.arange(32, dtype=np.float32).reshape(2, 16)
    b = oracle.T5RelativePositionBias(table, num_buckets=16, max_distance=8, bidirectional=True)
    z = np.zeros((4, 4), np.float32)
    bk = oracle.masks.relative_position_bucket(_idx(4)[None, :] - _idx(4)[:, None], num_buckets=16,
                                               max_distance=8, bidirectional=True)
    for h in range(2):
        np.testing.assert_array_equal(b(z, h, _idx(4), _idx(4)), table[h][bk])
    max_d = 2
    t = np.arange(2 * max_d + 1, dtype=np.float32)
    lb = oracle.LearnedRelativePositionBias(t, max_distance=max_d)
    rel = np.clip(_idx(5)[None, :] - _idx(3)[:, None], -max_d, max_d) + max_d
    np.testing.assert_array_equal(lb(np.zeros((3, 5), np.float32), 0, _idx(3), _idx(5)), t[rel])
