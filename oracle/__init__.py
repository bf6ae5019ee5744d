"""CPU oracle for the probjax fused-attention path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the algorithm of probjax's XLA attention
reference (``probjax/nn/pallas_kernels/kernels/attention_xla.py``) and the
pieces of the path that surround it (mask/bias objects, the split-KV
log-sum-exp merge, the latent-attention CPU path, rotary encoding).  Every
function cites the reference file:line it follows.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker or the timed CPU
baseline.  The product package ``probjax_amd`` never imports it: the HIP path
fails loudly when its library is missing instead of falling back here.

Pinning status of each function is recorded in the module docstrings
(``parity pinned by ...``); nothing here is "parity unpinned".
"""

from .bf16 import round_bf16, round_f16, round_to  # noqa: F401
from .masks import (  # noqa: F401
    BlockDiagonalCausalMask,
    BlockDiagonalMask,
    CausalAlibiBias,
    CausalFromBottomRightMask,
    CausalLocalWindowMask,
    CausalMask,
    ComposeMask,
    ConstantBias,
    DenseBias,
    DistanceDecayBias,
    IdentityBias,
    KVLenMask,
    LocalWindowMask,
    NoMask,
    PerHeadScaleBias,
    PrefixLMMask,
    QKVLengthMask,
    SameSegmentMask,
    KeyPaddingMask,
    LowRankBias,
    BatchedLowRankBias,
    LearnedAlibiBias,
    LearnedRelativePositionBias,
    MarginalizationMask,
    NotMask,
    T5RelativePositionBias,
    SeqLenMask,
    SoftCappingBias,
    SumBias,
    SymmetricAlibiBias,
)
from .attention_xla import auto_strategy, xla_attention  # noqa: F401
from .splitkv import default_num_splits, splitkv_forward  # noqa: F401
from .latent import materialize_kv, materialized_mla, materialized_mla_backward, xla_mla  # noqa: F401
from .rope import apply_rotary, inv_freq  # noqa: F401
from .lowrank import fold_low_rank, flex_low_rank, flex_low_rank_backward, split_low_rank_bias  # noqa: F401
