"""pjx_splitkv_decode_static (the split-KV decode whose partials live in the
library's own device array, for callers that cannot allocate) against
pjx_splitkv_decode with a caller workspace, through the C ABI: the same
kernels on the same inputs give bit-identical outputs and LSE.  Two calls in
a row, the second smaller (the array keeps the first call's contents, which
the second must not read), then a size past the array is refused.
"""

import ctypes
import math

import numpy as np
import pytest

from tests._helpers import rng_normal, to_dev

pytestmark = pytest.mark.gpu


def _call_both(device, B, S, Hq, Hkv, D, Lq, lengths, seed):
    import torch
    from probjax_amd import native

    lib = native.load()
    q, k, v = rng_normal(seed, (B, Lq, Hq, D), (B, S, Hkv, D), (B, S, Hkv, D))
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    L = torch.from_numpy(np.asarray(lengths, np.int32)).to(device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    scale = 1.0 / math.sqrt(D)
    rows = (Hq // Hkv) * Lq
    outs = []
    for static in (False, True):
        o = torch.full((B, Lq, Hq, D), float("nan"), dtype=torch.bfloat16, device=device)
        lse = torch.full((B, Hq, Lq), float("nan"), dtype=torch.float32, device=device)
        ptrs = [ctypes.c_void_p(t.data_ptr()) for t in (tq, tk, tv, L, o, lse)]
        if static:
            rc = lib.pjx_splitkv_decode_static(native.PJX_DTYPE_BF16, *ptrs, B, Lq, S, Hq, Hkv, D, D, scale, 0,
                                               stream)
        else:
            nbytes = int(lib.pjx_decode_workspace_size(B, Hkv, rows, S, D, 0))
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            rc = lib.pjx_splitkv_decode(native.PJX_DTYPE_BF16, *ptrs, ctypes.c_void_p(ws.data_ptr()), nbytes,
                                        B, Lq, S, Hq, Hkv, D, D, scale, 0, stream)
        native.check(rc)
        torch.cuda.synchronize()
        outs.append((o, lse))
    return outs


def test_static_decode_matches_workspace_decode_twice(device):
    import torch

    cases = [
        # B, S, Hq, Hkv, D, Lq, lengths
        (8, 4096, 32, 8, 128, 1, [4096, 17, 0, 2048, 3000, 4095, 1, 2049]),
        (2, 1000, 8, 2, 64, 2, [1000, 333]),
    ]
    for i, (B, S, Hq, Hkv, D, Lq, lengths) in enumerate(cases):
        print(f"static decode call {i}: B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} Lq={Lq}", flush=True)
        (o_ws, l_ws), (o_st, l_st) = _call_both(device, B, S, Hq, Hkv, D, Lq, lengths, 500 + i)
        assert not torch.isnan(o_st.float()).any()
        assert torch.equal(o_ws, o_st)
        assert torch.equal(l_ws, l_st)  # +inf for the empty sequence in both


def test_static_decode_refuses_sizes_past_its_array(device):
    import torch
    from probjax_amd import native

    lib = native.load()
    B, S, Hq, Hkv, D = 256, 1 << 20, 16, 16, 128
    need = int(lib.pjx_decode_workspace_size(B, Hkv, 1, S, D, 0))
    assert need > native.PJX_DECODE_STATIC_SCRATCH_BYTES
    # the size check runs before any pointer is used or kernel launched; with
    # null pointers a regression past it would be refused, not launched
    rc = lib.pjx_splitkv_decode_static(native.PJX_DTYPE_BF16, None, None, None, None, None, None,
                                       B, 1, S, Hq, Hkv, D, D, 0.1, 0,
                                       ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream))
    assert rc == 3
    assert "scratch" in lib.pjx_last_error().decode()
