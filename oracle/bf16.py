"""bfloat16 rounding for the numpy oracle (numpy has no bf16 dtype).

Values are kept in float32 arrays; ``round_bf16`` rounds them to the nearest
bfloat16 (ties to even), which is what ``x.astype(jnp.bfloat16)`` does in the
reference (e.g. ``attention_xla.py:349`` casting P to V's dtype, ``:679``
casting the output to q's dtype).  Pinned by exact known values in
``tests/test_oracle_basics.py`` (1 + 2^-8 ties to 1, 1 + 3*2^-8 ties up,
NaN/inf preserved) and against ``torch.bfloat16`` conversion.
"""

import numpy as np


def round_bf16(x):
    """Round float32 values to the nearest bfloat16 (RNE); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> np.uint64(16)) & np.uint64(1)
    r = ((u + np.uint64(0x7FFF) + lsb) >> np.uint64(16)) << np.uint64(16)
    out = (r & np.uint64(0xFFFFFFFF)).astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(x.shape)
