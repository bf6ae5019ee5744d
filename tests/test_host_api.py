"""Host-side logic of the probjax-API mirror (no GPU needed).

Restates the reference's dispatch tests where they apply to this path:
``use_splitkv`` only for exact cases (probjax tests/test_attention_gqa_splitkv.py:
224-232), route functions returning None to fall through and forced backends
raising ValueError (tests/test_attention_device_defaults.py:25-59), the
argument checks of ``flex_attention`` / ``mla``.
"""

import numpy as np
import pytest
import torch

from probjax_amd import attention as A
from probjax_amd import masks as M


def _qkv(b=1, lq=1, lk=2048, hq=4, hkv=2, d=128, dtype=torch.bfloat16):
    return (torch.zeros(b, lq, hq, d, dtype=dtype), torch.zeros(b, lk, hkv, d, dtype=dtype),
            torch.zeros(b, lk, hkv, d, dtype=dtype))


def test_lower_mask_table():
    assert M.lower_mask(None) == M.LoweredMask()
    assert M.lower_mask(M.NoMask()) == M.LoweredMask()
    assert M.lower_mask(M.CausalMask()).causal
    lm = M.lower_mask(M.CausalMask() & M.KVLenMask([3, 4]))
    assert lm.causal and list(lm.kv_lengths) == [3, 4]
    lm = M.lower_mask(M.QKVLengthMask(5, 7) & M.QKVLengthMask(6, 3))
    assert (lm.q_valid, lm.kv_valid) == (5, 3)
    assert M.lower_mask(M.CausalMask() | M.KVLenMask([1])) is None  # OR is not an AND of kernel masks


def test_lower_mask_accepts_foreign_objects_by_name():
    class CausalMask:  # noqa: D401 - stands for probjax's own class
        pass

    class KVLenMask:
        def __init__(self, L):
            self.kv_lengths = L

    assert M.lower_mask(CausalMask()).causal
    assert M.lower_mask(KVLenMask([2])).kv_lengths == [2]

    class MarginalizationMask:
        pass

    assert M.lower_mask(MarginalizationMask()) is None


def test_lower_bias():
    b = torch.zeros(1, 2, 3, 4)
    assert M.lower_bias(None) is None
    assert M.lower_bias(M.DenseBias(b)).dense is b
    assert M.lower_bias(object()) is False
    with pytest.raises(ValueError):
        M.DenseBias(torch.zeros(3, 4))


def test_compose_two_stateful_raises():
    with pytest.raises(ValueError, match="Cannot compose two stateful masks"):
        M.ComposeMask("and", M.KVLenMask([1]), M.KVLenMask([2]))


def test_use_splitkv_only_for_exact_cases():
    q, k, _ = _qkv()
    assert not A.use_splitkv(q, k, split_kv=False)
    assert not A.use_splitkv(q, k, mask=M.CausalMask(), split_kv=True)
    assert not A.use_splitkv(q, k, dropout_rate=0.1, split_kv=True)
    assert not A.use_splitkv(q, k, bias=M.DenseBias(torch.zeros(1, 1, 1, 2048)), split_kv=True)
    assert A.use_splitkv(q, k)                                  # Lq <= 64, Lkv >= 1024
    assert A.use_splitkv(q, k, mask=M.KVLenMask([5]))           # exact with lengths too
    q2, k2, _ = _qkv(lk=512)
    assert not A.use_splitkv(q2, k2) and A.use_splitkv(q2, k2, split_kv=True)
    q3, k3, _ = _qkv(lq=100)
    assert not A.use_splitkv(q3, k3)
    q4, k4, _ = _qkv(hq=64, hkv=2)                              # 32 rows per KV head
    assert A.use_splitkv(q4, k4, split_kv=True)
    q4b, k4b, _ = _qkv(hq=64, hkv=2, lq=3)                      # 96 rows: two row groups
    assert A.use_splitkv(q4b, k4b, split_kv=True)
    q5, k5, _ = _qkv(dtype=torch.float32)
    assert A.use_splitkv(q5, k5)                                # fp32 split-KV
    q5b, k5b, _ = _qkv(dtype=torch.float32, hq=64, hkv=1)       # 64 fp32 rows: two row groups
    assert A.use_splitkv(q5b, k5b, split_kv=True)
    # head dims up to 256 are zero-padded to a kernel width; wider ones are not
    q6, k6 = torch.zeros(1, 1, 8, 96, dtype=torch.bfloat16), torch.zeros(1, 2048, 2, 96, dtype=torch.bfloat16)
    assert A.use_splitkv(q6, k6)
    q7, k7 = torch.zeros(1, 1, 8, 160, dtype=torch.bfloat16), torch.zeros(1, 2048, 2, 160, dtype=torch.bfloat16)
    assert A.use_splitkv(q7, k7, split_kv=True)
    q8, k8 = torch.zeros(1, 1, 8, 300, dtype=torch.bfloat16), torch.zeros(1, 2048, 2, 300, dtype=torch.bfloat16)
    assert not A.use_splitkv(q8, k8, split_kv=True)


def test_kernel_width_and_padding():
    ds = (1, 32, 64, 65, 96, 128, 129, 256, 257)
    assert [A._kernel_width(d) for d in ds] == [64, 64, 64, 128, 128, 128, 256, 256, None]
    assert [A._kernel_width(d, torch.float32) for d in ds] == [64, 64, 64, 128, 128, 128, 256, 256, None]
    assert [A._decode_width(d) for d in ds] == [64, 64, 64, 128, 128, 128, 256, 256, None]
    assert [A._latent_width(r, torch.bfloat16) for r in (100, 200, 300, 512, 513, 576, 577)] == \
        [128, 256, 512, 512, 576, 576, None]
    assert [A._latent_width(r, torch.float32) for r in (100, 200, 300, 576)] == [128, 256, None, None]
    x = torch.randn(2, 3, 4, 40, requires_grad=True)
    y = A._pad_features(x, 64)
    assert y.shape == (2, 3, 4, 64) and torch.equal(y[..., :40], x) and not y[..., 40:].any()
    y.sum().backward()
    assert x.grad.shape == x.shape


def test_route_falls_through_off_device():
    q, k, v = _qkv()
    assert A.hip_attention_or_none(q, k, v, mask=None, bias=None, dropout_rate=0.0, sm_scale=0.1) is None
    assert A.hip_attention_or_none(q, k, v, mask=None, bias=None, dropout_rate=0.0, sm_scale=0.1,
                                   force=True) is None


def test_route_respects_env_switch(monkeypatch):
    q, k, v = _qkv()
    monkeypatch.setenv("PROBJAX_ATTENTION_HIP", "0")
    assert not A.device_table_enabled()
    assert A.hip_attention_or_none(q, k, v, mask=None, bias=None, dropout_rate=0.0, sm_scale=0.1) is None
    monkeypatch.setenv("PROBJAX_ATTENTION_HIP", "1")
    assert A.device_table_enabled()


def test_eligibility_rejects_without_touching_a_device(monkeypatch):
    """Shapes/dtypes/masks the kernels do not take make the route fall through."""
    monkeypatch.setattr(A, "hip_device", lambda t: True)
    q, k, v = _qkv()
    assert A._eligible(q, k, v, mask=None, bias=None, dropout_rate=0.1) is None
    class Unknown(M.AttentionMask):
        pass

    assert A._eligible(q, k, v, mask=Unknown(), bias=None, dropout_rate=0.0) is None
    # an OR composition has no in-kernel form: it becomes a 0 / -inf dense bias
    q4, k4, v4 = _qkv(lq=4, lk=4)
    lm, lb = A._eligible(q4, k4, v4, mask=M.CausalMask() | M.LocalWindowMask(1, 0), bias=None, dropout_rate=0.0)
    want = torch.where(torch.tril(torch.ones(4, 4, dtype=torch.bool)), 0.0, float("-inf"))
    assert lm == M.LoweredMask() and lb.dense.shape == (1, 1, 4, 4) and torch.equal(lb.dense[0, 0], want)
    assert A._eligible(q, k, v, mask=None, bias=object(), dropout_rate=0.0) is None
    assert A._eligible(q, k, v[:, :5], mask=None, bias=None, dropout_rate=0.0) is None
    assert A._eligible(q, k, v, mask=M.KVLenMask([1, 2]), bias=None, dropout_rate=0.0) is None  # B = 1
    lm, b = A._eligible(q, k, v, mask=M.KVLenMask([7]), bias=None, dropout_rate=0.0)
    assert lm.kv_lengths.dtype == torch.int32 and b is None
    q64 = q.to(torch.float64)
    assert A._flash_plan(q64, k, v, M.LoweredMask(), None) is None
    q16, k16, v16 = (t.to(torch.float16) for t in (q, k, v))
    assert A._flash_plan(q16, k16, v16, M.LoweredMask(), None) is not None
    assert A._decode_plan(q16, k16, v16, M.LoweredMask(), None) is not None
    q96 = torch.zeros(1, 4, 4, 96, dtype=torch.bfloat16)
    assert A._flash_plan(q96, q96, q96, M.LoweredMask(), None) is None


def test_bias_sums_lower_to_one_dense_term(monkeypatch):
    """Several dense terms of a SumBias (any broadcast shapes) become one
    tensor, a second distance term its dense values; a term that does not
    broadcast to [B, Hq, Lq, Lk] makes the route fall through."""
    monkeypatch.setattr(A, "hip_device", lambda t: True)
    q, k = torch.zeros(2, 8, 2, 64), torch.zeros(2, 10, 2, 64)
    b1, b2 = torch.randn(1, 2, 8, 10), torch.randn(2, 1, 8, 10)
    _, lb = A._eligible(q, k, k, mask=None, bias=M.DenseBias(b1) + M.DenseBias(b2), dropout_rate=0.0)
    assert torch.equal(lb.dense, b1 + b2)
    _, lb = A._eligible(q, k, k, mask=None, bias=M.CausalAlibiBias() + M.DistanceDecayBias(0.5), dropout_rate=0.0)
    assert lb.alibi == "causal" and torch.equal(lb.dense, M.dense_distance("decay", 0.5, 2, 8, 10, "cpu"))
    bad = M.DenseBias(b1) + M.DenseBias(torch.zeros(3, 1, 8, 10))
    assert A._eligible(q, k, k, mask=None, bias=bad, dropout_rate=0.0) is None


def test_flex_attention_argument_checks():
    q, k, v = _qkv(hq=4, hkv=2)
    with pytest.raises(ValueError, match="same dtype"):
        A.flex_attention(q, k.float(), v)
    with pytest.raises(ValueError, match="at least 3 dimensional"):
        A.flex_attention(q[0, 0], k, v)
    with pytest.raises(ValueError, match="enable_gqa=True"):
        A.flex_attention(q, k, v)
    q3, k3, v3 = _qkv(hq=3, hkv=2)
    with pytest.raises(ValueError, match="multiple of kv heads"):
        A.flex_attention(q3, k3, v3, enable_gqa=True)
    with pytest.raises(ValueError, match="implementation must be"):
        A.flex_attention(q, k, v, enable_gqa=True, implementation="triton")
    # off a gfx950 device the forced route refuses (no CPU fallback)
    with pytest.raises(ValueError, match="cannot compute this call exactly"):
        A.flex_attention(q, k, v, enable_gqa=True, implementation="hip")


def test_mha_and_mla_refuse_off_device():
    q, k, v = _qkv()
    with pytest.raises(ValueError, match="ROCm device"):
        A.mha(q, k, v)
    _, k3, v3 = _qkv(hkv=3)
    with pytest.raises(ValueError, match="multiple of KV heads"):
        A.mha(q, k3, v3)
    qm = torch.zeros(2, 1, 16, 576, dtype=torch.bfloat16)
    c = torch.zeros(2, 64, 576, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        A.mla(qm, c)
    with pytest.raises(ValueError, match="rank 4"):
        A.mla(qm[0], c)
    with pytest.raises(ValueError, match="batch mismatch"):
        A.mla(qm, c[:1])
    with pytest.raises(ValueError, match="both wk and wv"):
        A.mla(qm, c, wk=torch.zeros(16, 576, 576))
    with pytest.raises(ValueError, match="qk_head_dim == kv_lora_rank"):
        A.mla(qm[..., :512], c)
    # materialised mode: the reference's shape checks (latent_attention.py:690-701)
    qd = torch.zeros(2, 4, 16, 96, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="wk must be"):
        A.mla(qd, c, torch.zeros(16, 64, 576), torch.zeros(16, 64, 576))
    with pytest.raises(ValueError, match="wv must be"):
        A.mla(qd, c, torch.zeros(16, 96, 576), torch.zeros(16, 64, 512))
    wk, wv = torch.zeros(16, 96, 576, dtype=torch.bfloat16), torch.zeros(16, 64, 576, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm device"):
        A.mla(qd, c, wk, wv)
    with pytest.raises(ValueError, match="head dims up to 256"):
        A.mla(torch.zeros(2, 4, 16, 300), c.float(), torch.zeros(16, 300, 576), torch.zeros(16, 128, 576))
    with pytest.raises(ValueError, match="no dropout"):
        A.mla(qd, c, wk, wv, dropout_rate=0.1)


def test_dot_product_attention_array_masks_need_the_device():
    q, k, v = _qkv()
    with pytest.raises(ValueError, match="ROCm device"):
        A.dot_product_attention(q, k, v, mask=torch.ones(1, 1, 1, 2048, dtype=torch.bool))
    with pytest.raises(ValueError, match="broadcast"):
        A.dot_product_attention(q, k, v, bias=torch.zeros(3, 1, 1, 2048))


def test_splitkv_forward_num_splits_to_chunk(monkeypatch):
    seen = {}

    def fake(q, k, v, *, sm_scale, kv_lengths, chunk, return_lse):
        seen["chunk"] = chunk
        return q

    monkeypatch.setattr(A.hip, "splitkv_decode", fake)
    q, k, v = _qkv(lk=1000)
    A.splitkv_forward(q, k, v, sm_scale=0.1, num_splits=3)
    assert seen["chunk"] == 384  # ceil(1000/3) = 334 -> 3 x 128
    A.splitkv_forward(q, k, v, sm_scale=0.1)
    assert seen["chunk"] == 0
    # a 48-wide head runs the kernel at 64 and comes back 48 wide
    q48, k48, v48 = (x[..., :48] for x in (q, k, v))
    out = A.splitkv_forward(q48, k48, v48, sm_scale=0.1)
    assert out.shape[-1] == 48
    with pytest.raises(ValueError):
        A.splitkv_forward(q, k, v, sm_scale=0.1, num_splits=0)
    assert np.isclose(A._SPLITKV_MIN_KV_LEN, 1024)


def test_lower_extended_masks():
    """Positional masks lower to intersected intervals; stateful ones carry data."""
    lm = M.lower_mask(M.CausalMask() & M.LocalWindowMask(5, 2))
    assert (lm.causal_shift, lm.window_left, lm.window_right) == (0, 5, 2) and lm.extended
    lm = M.lower_mask(M.LocalWindowMask(4) & M.CausalLocalWindowMask(3))
    assert (lm.window_left, lm.window_right) == (3, 0)
    lm = M.lower_mask(M.CausalFromBottomRightMask(3, 10) & M.CausalMask())
    assert lm.causal_shift == 0  # k <= q + 7 and k <= q  ->  k <= q
    assert M.lower_mask(M.CausalFromBottomRightMask(3, 10)).causal_shift == 7
    assert not M.lower_mask(M.CausalMask()).extended
    lm = M.lower_mask(M.PrefixLMMask([2, 3]) & M.QKVLengthMask(5, 6))
    assert lm.prefix_lengths == [2, 3] and lm.q_valid == 5 and not lm.causal
    lm = M.lower_mask(M.BlockDiagonalCausalMask([0, 0, 1]))
    assert lm.segment_q == [0, 0, 1] and lm.segment_k is None and lm.causal_shift == 0
    assert M.lower_mask(M.SeqLenMask([3])).seq_lengths == [3]
    with pytest.raises(ValueError):
        M.SameSegmentMask([0]) & M.KVLenMask([1])
    assert M.lower_mask(M.LocalWindowMask(-1)) is None


def test_lower_score_modifiers():
    lb = M.lower_bias(M.SymmetricAlibiBias() + M.ConstantBias(0.5) + M.ConstantBias(0.25) + M.IdentityBias())
    assert lb.alibi == "symmetric" and lb.constant == 0.75 and lb.dense is None and lb.extended
    lb = M.lower_bias(M.DistanceDecayBias(0.3) + M.DenseBias(torch.zeros(1, 1, 2, 2)))
    assert lb.alibi == "decay" and lb.alibi_alpha == 0.3 and lb.dense is not None
    assert M.lower_bias(M.SoftCappingBias(30.0)).softcap == 30.0
    assert M.lower_bias(M.PerHeadScaleBias([1.0, 2.0])).head_scales.tolist() == [1.0, 2.0]
    # a non-additive modifier inside a sum: not taken
    assert M.lower_bias(M.SoftCappingBias(5.0) + M.ConstantBias(1.0)) is False
    # two dense biases, or a second distance term: the first stays in the
    # kernel, the rest are added to the dense bias per call
    d = M.DenseBias(torch.zeros(1, 1, 2, 2))
    lb = M.lower_bias(d + d)
    assert lb.dense is not None and len(lb.dense_more) == 1
    lb = M.lower_bias(M.CausalAlibiBias() + M.SymmetricAlibiBias() + M.DistanceDecayBias(0.2))
    assert lb.alibi == "causal" and lb.distance == [("symmetric", 1.0), ("decay", 0.2)]


def test_dense_distance_matches_oracle():
    import numpy as np

    import oracle

    for lq, lk in ((5, 5), (3, 9), (9, 2)):
        for kind, mine in (("causal", oracle.CausalAlibiBias()), ("symmetric", oracle.SymmetricAlibiBias()),
                           ("decay", oracle.DistanceDecayBias(0.37))):
            got = M.dense_distance(kind, 0.37, 3, lq, lk, "cpu")[0]
            assert got.shape[-2:] == (lq, lk) and got.shape[0] in (1, 3)
            for h in range(3):
                want = mine(np.zeros((lq, lk), np.float32), h, np.arange(lq), np.arange(lk))
                np.testing.assert_allclose(got[h if got.shape[0] == 3 else 0].numpy(), want, rtol=0, atol=1e-6)


def test_score_mods_arguments():
    lm = M.lower_mask(M.CausalFromBottomRightMask(4, 6) & M.SameSegmentMask([0, 0, 1, 1]))
    # segment ids per position: the key ids default to the query ids, so Lq == Lk is needed
    assert A._score_mods(lm, None, 2, 4, 6, 3, "cpu") is False
    lm = M.lower_mask(M.CausalFromBottomRightMask(4, 4) & M.SameSegmentMask([0, 0, 1, 1]))
    m = A._score_mods(lm, M.lower_bias(M.CausalAlibiBias()), 2, 4, 4, 3, "cpu")
    assert m.causal_shift == 0 and m.segment_q.shape == (2, 4) and m.segment_k.dtype == torch.int32
    assert torch.allclose(m.alibi_slopes, torch.tensor([0.5, 0.25, 0.125])) and not m.alibi_symmetric
    m = A._score_mods(M.lower_mask(M.PrefixLMMask(3)), M.lower_bias(M.PerHeadScaleBias([2.0])), 2, 4, 4, 3, "cpu")
    assert m.prefix_lengths.tolist() == [3, 3] and m.head_scales.tolist() == [2.0, 2.0, 2.0]
    assert A._score_mods(M.lower_mask(M.CausalMask()), None, 1, 4, 4, 1, "cpu") is None


def test_key_padding_lowering():
    """KeyPaddingMask carries a per-row key count: [T] shared by every batch,
    [B, T] per batch, rows past T count 0; one query row folds to per-batch
    lengths (the split-KV route)."""
    lm = M.lower_mask(M.KeyPaddingMask([4, 2]) & M.CausalMask())
    assert lm.extended and lm.row_kv_lengths == [4, 2] and lm.causal_shift == 0
    with pytest.raises(ValueError):
        M.KeyPaddingMask([1]) & M.KVLenMask([1])
    rows = A._row_kv_lengths(torch.tensor([4, 2]), 3, 3, "cpu")
    assert rows.tolist() == [[4, 2, 0]] * 3 and rows.dtype == torch.int32
    assert A._row_kv_lengths(torch.tensor([[5, 6, 7], [1, 2, 3]]), 2, 2, "cpu").tolist() == [[5, 6], [1, 2]]
    assert A._row_kv_lengths(7, 2, 3, "cpu").tolist() == [[7, 7, 7]] * 2
    assert A._row_kv_lengths(torch.tensor([True, False]), 1, 2, "cpu").tolist() == [[1, 0]]
    assert A._row_kv_lengths(torch.tensor([1.5]), 1, 1, "cpu") is None
    assert A._row_kv_lengths(torch.ones(3, 2, dtype=torch.int32), 2, 2, "cpu") is None  # batch mismatch
    m = A._score_mods(M.LoweredMask(row_kv_lengths=rows), None, 3, 3, 5, 2, "cpu")
    assert m.row_kv_lengths is rows and m.segment_q is None
    q = torch.zeros(2, 1, 8, 128, dtype=torch.bfloat16)
    k = torch.zeros(2, 4096, 8, 128, dtype=torch.bfloat16)
    assert A.use_splitkv(q, k, mask=M.KeyPaddingMask(torch.tensor([9, 9])))
    assert not A.use_splitkv(torch.zeros(2, 2, 8, 128, dtype=torch.bfloat16), k, mask=M.KeyPaddingMask([9, 9]))


def test_mla_absorb_rule():
    """probjax's FLOP rule (latent_attention.py:616-620): decoding absorbs,
    full-length prefill with a wide latent materialises."""
    assert A._absorbed_cheaper(1, 4096, 512, 128, 128)
    assert not A._absorbed_cheaper(4096, 4096, 512, 128, 128)
    assert A._absorbed_cheaper(4096, 4096, 64, 128, 128)  # narrow latent


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_low_rank_fold_matches_oracle(dtype):
    """The mirror's factor layouts and folding (torch, no kernels) against the
    oracle's restatement of flex_attention:1600-1635."""
    import numpy as np

    import oracle
    from oracle.lowrank import fold_low_rank

    rng = np.random.default_rng(0)
    B, L, Hq, Hkv, D = 2, 12, 4, 2, 16
    q, k, v = (rng.standard_normal(s).astype(np.float32) for s in ((B, L, Hq, D), (B, L, Hkv, D), (B, L, Hkv, D)))
    qf, kf = (rng.standard_normal((Hq, 14, 3)).astype(np.float32) for _ in range(2))
    kb = rng.standard_normal((B, L)).astype(np.float32)
    slopes = np.array([0.5, 0.25, 0.125, 0.0625], np.float32)
    mine = [M.LowRankBias(torch.from_numpy(qf), torch.from_numpy(kf), scale=0.5),
            M.BatchedLowRankBias.from_key_bias(torch.from_numpy(kb)),
            M.LearnedAlibiBias(torch.from_numpy(slopes), key_offset=2)]
    theirs = [oracle.LowRankBias(qf, kf, scale=0.5), oracle.BatchedLowRankBias.from_key_bias(kb),
              oracle.LearnedAlibiBias(slopes, key_offset=2)]
    terms, rest = M.split_low_rank_bias(mine[0] + M.CausalAlibiBias() + mine[1] + mine[2])
    assert [type(t).__name__ for t in terms] == ["LowRankBias", "BatchedLowRankBias", "LearnedAlibiBias"]
    assert type(rest).__name__ == "CausalAlibiBias"
    tq, tk, tv = (torch.from_numpy(x).to(dtype) for x in (q, k, v))
    q2, k2, v2, out_dim = A._fold_low_rank(tq, tk, tv, terms, 0.25)
    assert out_dim == D and q2.shape[-1] == 64 and k2.shape == (B, L, Hq, 64)
    dt = "bf16" if dtype == torch.bfloat16 else "f32"
    wq, wk, wv = fold_low_rank(q, k, v, theirs, 0.25, dt)
    n = wq.shape[-1]
    for got, want in ((q2, wq), (k2, wk), (v2, wv)):
        np.testing.assert_allclose(got[..., :n].float().numpy(), want, rtol=0, atol=1e-6)
        assert not got[..., n:].float().any()
    with pytest.raises(ValueError, match="positive sm_scale"):
        A._fold_low_rank(tq, tk, tv, terms, 0.0)
    assert A._fold_low_rank(torch.zeros(1, 4, 4, 256), torch.zeros(1, 4, 4, 256), torch.zeros(1, 4, 4, 256),
                            terms[:1], 0.1) is None
    with pytest.raises(ValueError, match="same rank"):
        M.LowRankBias(torch.zeros(2, 4, 3), torch.zeros(2, 4, 2))


def _mask_pairs(B, lq, lk):
    """(mirror mask, oracle mask) pairs over every mask class of the path."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(3)
    lens = rng.integers(0, lk + 1, size=B).astype(np.int32)
    seg_q = np.sort(rng.integers(0, 3, size=(B, lq)), axis=1).astype(np.int32)
    marg = rng.random((B, lq)) < 0.6
    kl = rng.integers(0, lk + 1, size=lq - 2).astype(np.int32)
    t = torch.from_numpy
    return [
        (M.CausalMask(), oracle.CausalMask()),
        (M.CausalFromBottomRightMask(lq, lk), oracle.CausalFromBottomRightMask(lq, lk)),
        (M.LocalWindowMask(2, 1), oracle.LocalWindowMask(2, 1)),
        (M.CausalLocalWindowMask(3), oracle.CausalLocalWindowMask(3)),
        (M.QKVLengthMask(lq - 1, lk - 2), oracle.QKVLengthMask(lq - 1, lk - 2)),
        (M.KVLenMask(t(lens)), oracle.KVLenMask(lens)),
        (M.PrefixLMMask(t(lens)), oracle.PrefixLMMask(lens)),
        (M.SeqLenMask(t(lens)), oracle.SeqLenMask(lens)),
        (M.KeyPaddingMask(t(kl)), oracle.KeyPaddingMask(kl)),
        (M.MarginalizationMask(t(marg)), oracle.MarginalizationMask(marg)),
        (~M.CausalMask(), ~oracle.CausalMask()),
        (M.CausalMask() | M.LocalWindowMask(1, 2), oracle.CausalMask() | oracle.LocalWindowMask(1, 2)),
        (M.CausalMask() ^ M.KVLenMask(t(lens)), oracle.CausalMask() ^ oracle.KVLenMask(lens)),
        (~(M.MarginalizationMask(t(marg)) & M.CausalMask()),
         ~(oracle.MarginalizationMask(marg) & oracle.CausalMask())),
    ] + ([(M.SameSegmentMask(t(seg_q)), oracle.SameSegmentMask(seg_q)),
          (M.BlockDiagonalCausalMask(t(seg_q)), oracle.BlockDiagonalCausalMask(seg_q))] if lq == lk else [])


@pytest.mark.parametrize("lq,lk", [(6, 6), (5, 9)])
def test_dense_keep_matches_oracle(lq, lk):
    """The dense forms the route falls back to agree with the oracle's tile
    evaluation of every mask class (stateful payloads included)."""
    import numpy as np

    B = 2
    for mine, theirs in _mask_pairs(B, lq, lk):
        got = M.dense_keep(mine, B, lq, lk, "cpu")
        want = np.stack([theirs.tile_keep(b, np.arange(lq), np.arange(lk)) for b in range(B)])
        assert got is not None and got.shape == (B, lq, lk), type(mine).__name__
        np.testing.assert_array_equal(got.numpy(), want, err_msg=type(mine).__name__)
        assert M.dense_supported(mine)


def test_dense_relpos_matches_oracle():
    import numpy as np

    import oracle

    rng = np.random.default_rng(4)
    for lq, lk in ((7, 7), (3, 40)):
        t5 = rng.standard_normal((3, 16)).astype(np.float32)
        lr = rng.standard_normal((1, 9)).astype(np.float32)
        pairs = [(M.T5RelativePositionBias(torch.from_numpy(t5), num_buckets=16, max_distance=10),
                  oracle.T5RelativePositionBias(t5, num_buckets=16, max_distance=10)),
                 (M.T5RelativePositionBias(torch.from_numpy(t5[:1]), num_buckets=16, max_distance=20,
                                           bidirectional=False),
                  oracle.T5RelativePositionBias(t5[:1], num_buckets=16, max_distance=20, bidirectional=False)),
                 (M.LearnedRelativePositionBias(torch.from_numpy(lr), max_distance=4),
                  oracle.LearnedRelativePositionBias(lr, max_distance=4))]
        for mine, theirs in pairs:
            got = M.dense_relpos(mine, lq, lk, "cpu")[0]
            for h in range(got.shape[0]):
                want = theirs(np.zeros((lq, lk), np.float32), h, np.arange(lq), np.arange(lk))
                np.testing.assert_array_equal(got[h].numpy(), want)


def test_flax_array_mask_and_bias_lowering():
    q, k = torch.zeros(6, 5, 4, 8), torch.zeros(6, 7, 2, 8)
    mask = torch.ones(3, 1, 5, 7, dtype=torch.bool)  # batch dims (2, 3) broadcast over the first
    mask[1, 0, 2] = False                              # row 2 of batch (*, 1) drops every key
    mask[0, 0, 0, 3] = False
    bias = torch.randn(4, 5, 7, requires_grad=True)
    m, b = A._flax_arrays(mask, bias, (2, 3), q, k)
    assert m is None and isinstance(b, M.DenseBias) and b.bias.shape == (6, 4, 5, 7)
    d = b.bias
    assert torch.isinf(d[1, :, 2]).all() and torch.isinf(d[4, :, 2]).all() and torch.isinf(d[0, :, 0, 3]).all()
    fin = torch.isfinite(d)
    assert torch.equal(d[fin], bias.expand(6, 4, 5, 7)[fin])
    # an object mask stays; an object bias takes the array mask as one more term
    m2, b2 = A._flax_arrays(None, bias, (2, 3), q, k)
    assert b2.bias.requires_grad
    m3, b3 = A._flax_arrays(mask, None, (2, 3), q, k)
    assert b3.bias.shape == (6, 1, 5, 7)
    with pytest.raises(ValueError, match="heads"):
        A._flax_arrays(None, torch.zeros(3, 5, 7), (2, 3), q, k)
    with pytest.raises(ValueError, match="broadcast"):
        A._flax_arrays(None, torch.zeros(4, 4, 5, 7), (2, 3), q, k)


def test_flax_empty_rows_fill():
    """Rows with lse = +inf (no valid key) take the mean of V, per query head
    of each KV group; the others keep the kernel output.  No keys at all keep
    the zeros (Flax's einsum over an empty key axis)."""
    torch.manual_seed(0)
    B, Lq, Lk, Hq, Hkv, D = 2, 3, 5, 4, 2, 8
    out = torch.randn(B, Lq, Hq, D)
    v = torch.randn(B, Lk, Hkv, D)
    lse = torch.randn(B, Hq, Lq)
    lse[1, 3, 2] = float("inf")
    got = A._flax_empty_rows(out, lse, v)
    want = out.clone()
    want[1, 2, 3] = v[1, :, 1].mean(dim=0)
    assert torch.equal(got, want)
    v0 = torch.randn(B, 0, Hkv, D)
    lse0 = torch.full((B, Hq, Lq), float("inf"))
    z = torch.zeros(B, Lq, Hq, D)
    assert torch.equal(A._flax_empty_rows(z, lse0, v0), z)


def test_mla_decode_shape_rule():
    """The latent decode's (rank, v_dim) for a latent width and output width:
    the narrowest kernel rank that holds the width, then the narrowest output
    width that holds the requested columns."""
    assert A._mla_decode_shape(576, 512) == (576, 512)
    assert A._mla_decode_shape(576, 576) == (576, 576)
    assert A._mla_decode_shape(576, 300) == (576, 512)
    assert A._mla_decode_shape(512, 512) == (512, 512)
    assert A._mla_decode_shape(300, 300) == (512, 512)
    assert A._mla_decode_shape(200, 150) == (256, 256)
    assert A._mla_decode_shape(128, 128) == (128, 128)
    assert A._mla_decode_shape(40, 40) == (64, 64)
    assert A._mla_decode_shape(600, 512) is None


def test_ds_route_workspace_choice(monkeypatch):
    """flash_attention_bwd's workspace choice for the dS route: the larger
    workspace when the route exists and its dS fits the budget (or when asked
    for), the plain one otherwise; asking for a route that does not exist is a
    ValueError.  (No device is touched: the budget comes from the environment.)"""
    from probjax_amd import hip_attention as H

    monkeypatch.setenv("PJX_BWD_DS_MAX_BYTES", "1000")
    dev = "cpu"
    assert H._ds_route_bytes(100, 900, None, dev, "x") == 900
    assert H._ds_route_bytes(100, 1100, None, dev, "x") == 1100  # 1000 bytes of dS: within the budget
    assert H._ds_route_bytes(100, 1101, None, dev, "x") == 100  # 1001 bytes: the plain workspace
    assert H._ds_route_bytes(100, 1101, True, dev, "x") == 1101
    assert H._ds_route_bytes(100, 900, False, dev, "x") == 100
    assert H._ds_route_bytes(100, 0, None, dev, "x") == 100
    with pytest.raises(ValueError, match="no route"):
        H._ds_route_bytes(100, 0, True, dev, "no route")
