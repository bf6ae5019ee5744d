"""16-bit rounding for the numpy oracle (numpy has no bf16 dtype).

Values are kept in float32 arrays; ``round_bf16`` rounds them to the nearest
bfloat16 (ties to even), which is what ``x.astype(jnp.bfloat16)`` does in the
reference (e.g. ``attention_xla.py:349`` casting P to V's dtype, ``:679``
casting the output to q's dtype); ``round_f16`` likewise to IEEE binary16
(``x.astype(jnp.float16)``: ties to even, gradual underflow, overflow to
inf), through numpy's own float16.  ``round_to`` applies the rounding of the
emulated input dtype (``"bf16"``, ``"f16"``; ``"f32"`` leaves values alone).
Pinned by exact known values in ``tests/test_oracle_basics.py`` (bf16:
1 + 2^-8 ties to 1, 1 + 3*2^-8 ties up; f16: 1 + 2^-11 ties to 1,
1 + 3*2^-11 ties up, the smallest subnormal, 65520 -> inf; NaN/inf
preserved) and against ``torch.bfloat16`` / ``torch.float16`` conversion.
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


def round_f16(x):
    """Round float32 values to the nearest IEEE binary16 value (RNE); returns float32."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        return x.astype(np.float16).astype(np.float32)


LOW_PRECISION = ("bf16", "f16")


def round_to(x, dtype: str):
    """``x`` as a tensor of the emulated dtype holds it: rounded to bf16 or
    fp16; unchanged for ``"f32"``."""
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    if dtype != "f32":
        raise ValueError(f"unknown dtype {dtype!r} (expected 'f32', 'bf16' or 'f16')")
    return x
