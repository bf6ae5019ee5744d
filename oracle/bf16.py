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
    u = x.view(np.uint32)
    # u + 0x7FFF + lsb stays below 2^32 for every non-NaN bit pattern (the
    # largest, -inf/-max, is 0xFF800000 + 0x8000); NaNs are restored below.
    r = u + np.uint32(0x7FFF)
    r += (u >> np.uint32(16)) & np.uint32(1)
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(x.shape)
