"""Every kernel instance the 16-bit flash launchers can pick, each asserted and
checked against the oracle.

``pjx_flash_fwd`` (``launch_h16`` / ``launch_pipe128``) and ``pjx_flash_bwd``
(``run_bwd_h16``) choose a kernel instance from the head dim, the bias, the
extended masks and the grid size against the device's CU count.  Each case
below names the instance it must land on; the library's launch log
(``pjx_last_launches``) is asserted to hold exactly that instance, so a change
of thresholds cannot silently move a case to another kernel.

Grid sizes are large for the GPU but cheap for the oracle: many heads over
short sequences (e.g. 1 x 520 heads x 256 keys gives 1040 query tiles and
520 key blocks).  The instance names assume MI355X's 256 CUs for the
grid-size branches (asserted).

Tolerances (the bars of the other 16-bit tests): outputs max-abs <= 2e-2
against the fp32 oracle on the same 16-bit inputs, LSE max-abs <= 1e-2 where
finite and +inf exactly where the oracle's is; gradients within probjax's
gradient tolerance (tests/test_attention.py:597-626: atol 2e-2, rtol 1e-2)
against the oracle backward in the same 16-bit mode, dbias likewise, with atol
scaled by max(1, max|ref| / 4) as in the other backward tests: the kernels sum
a GQA group's dK / dV in fp32 before their one 16-bit rounding, where the
reference rounds each head's gradient and then sums, so with 4-8 heads per KV
head over causal rows the two differ by a few 16-bit steps of gradients that
reach ~6.
"""

import math

import numpy as np
import pytest

import oracle
from oracle.backward import attention_backward
from tests._helpers import max_abs, rng_normal, to_dev, to_np

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
FMT = {"bf16": "Bf16Fmt", "f16": "F16Fmt"}


def _round(x, dtype):
    return oracle.round_bf16(x) if dtype == "bf16" else oracle.round_f16(x)


def _tdt(dtype):
    import torch

    return torch.bfloat16 if dtype == "bf16" else torch.float16


def _require_256_cus():
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert cus == 256, f"the grid-size branches below are sized for 256 CUs, the device has {cus}"


def _launched():
    from probjax_amd import native

    return native.last_launches()


def _check_grad(got, want, what):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    atol = ATOL * max(1.0, float(np.max(np.abs(want), initial=0.0)) / 4.0)
    bad = err > atol + RTOL * np.abs(want)
    assert not bad.any(), (
        f"{what}: {int(bad.sum())} of {bad.size} outside atol {atol:.3g} rtol {RTOL}; "
        f"max err {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"
    )


def _omask(causal, lengths, L):
    m = oracle.CausalMask() if causal else None
    if lengths is not None:
        kl = oracle.KVLenMask(np.array(lengths, np.int32))
        m = kl if m is None else m & kl
    return m


# ---------------------------------------------------------------------------
# Forward: launch_h16 / launch_pipe128 without extended masks
# ---------------------------------------------------------------------------

FWD_CASES = {
    # name: D, B, Lq, Lk, Hq, Hkv, causal, kv_lengths, bias heads (None: no bias), instance
    # no bias, D = 128: two groups (<= 2 tiles per CU causal), 64-key (< 3 per CU), 32-key
    "pipe128_two_groups": (128, 1, 1000, 1000, 8, 2, True, None, None,
                           "flash_fwd_bf16_pipe_kernel<{E}, 128, 64, 2, 2>"),
    "pipe128_two_groups_noncausal": (128, 2, 384, 500, 8, 8, False, [500, 77], None,
                                     "flash_fwd_bf16_pipe_kernel<{E}, 128, 64, 2, 2>"),
    "pipe128_mid_causal": (128, 1, 256, 256, 300, 100, True, None, None,
                           "flash_fwd_bf16_pipe_kernel<{E}, 128, 64, 2, 1>"),
    "pipe128_mid_noncausal_kvlen": (128, 2, 256, 300, 100, 50, False, [300, 129], None,
                                    "flash_fwd_bf16_pipe_kernel<{E}, 128, 64, 2, 1>"),
    "pipe128_large": (128, 2, 300, 300, 160, 40, True, [300, 0], None,
                      "flash_fwd_bf16_pipe_kernel<{E}, 128, 32, 3, 1>"),
    # no bias, D = 64: two groups, else the 64-key kernel at any larger grid
    "pipe64_two_groups": (64, 1, 700, 700, 16, 4, True, None, None,
                          "flash_fwd_bf16_pipe_kernel<{E}, 64, 64, 2, 2>"),
    "pipe64_mid_causal": (64, 1, 256, 256, 300, 60, True, None, None,
                          "flash_fwd_bf16_pipe_kernel<{E}, 64, 64, 2, 1>"),
    "pipe64_large_noncausal": (64, 2, 384, 333, 200, 100, False, [333, 190], None,
                               "flash_fwd_bf16_pipe_kernel<{E}, 64, 64, 2, 1>"),
    # dense bias with 16-byte aligned rows: the LDS bias ring
    "ring128": (128, 2, 256, 256, 4, 2, True, [256, 100], 4, "flash_fwd_bf16_bias_ring_kernel<{E}, 128, 2>"),
    "ring64_three_groups": (64, 2, 256, 512, 4, 4, False, [512, 300], 1,
                            "flash_fwd_bf16_bias_ring_kernel<{E}, 64, 3>"),
    "ring64_two_groups": (64, 1, 128, 2100, 2, 1, False, [2000], 2,
                          "flash_fwd_bf16_bias_ring_kernel<{E}, 64, 2>"),
    # dense bias with unaligned rows (Lk % 4 != 0): bias in registers
    "regbias128": (128, 2, 200, 301, 4, 2, False, [301, 150], 4, "flash_fwd_bf16_kernel<{E}, 128, true, 0>"),
    "regbias64": (64, 1, 257, 257, 4, 4, True, None, 1, "flash_fwd_bf16_kernel<{E}, 64, true, 0>"),
}

GRID_SIZED = {"pipe128_two_groups", "pipe128_two_groups_noncausal", "pipe128_mid_causal",
              "pipe128_mid_noncausal_kvlen", "pipe128_large", "pipe64_two_groups", "pipe64_mid_causal",
              "pipe64_large_noncausal"}


# every case in bf16; the grid-sized no-bias instances in fp16 too (the bias
# kernels' fp16 forms are in test_gpu_fp16.py)
FWD_PARAMS = [(n, "bf16") for n in FWD_CASES] + [(n, "f16") for n in FWD_CASES if n in GRID_SIZED]


@pytest.mark.parametrize("name,dtype", FWD_PARAMS)
def test_forward_branch(device, name, dtype):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    D, B, Lq, Lk, Hq, Hkv, causal, lengths, bias_h, inst = FWD_CASES[name]
    if name in GRID_SIZED:
        _require_256_cus()
    expect = inst.format(E=FMT[dtype])
    print(f"fwd {name} {dtype}: D={D} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} causal={causal} "
          f"lengths={lengths} bias_heads={bias_h} -> {expect}", flush=True)
    q, k, v = (_round(x, dtype) for x in rng_normal(60, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D)))
    bias = None if bias_h is None else rng_normal(61, (1, bias_h, Lq, Lk), scale=0.5)[0]
    scale = 1.0 / math.sqrt(D)
    mask = _omask(causal, lengths, Lk)
    want, want_lse = oracle.xla_attention(q, k, v, mask=mask, bias=None if bias is None else oracle.DenseBias(bias),
                                          sm_scale=scale, dtype=dtype, return_lse=True)
    tdt = _tdt(dtype)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got, lse = flash_attention_fwd(*(to_dev(x, device, tdt) for x in (q, k, v)), sm_scale=scale, causal=causal,
                                   kv_lengths=L, bias=bt, return_lse=True)
    launched = _launched()
    torch.cuda.synchronize()
    assert launched == [expect], launched
    got, lse = to_np(got), to_np(lse)
    err = max_abs(got, want)
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= 2e-2
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-2
    dead = np.isposinf(want_lse).transpose(0, 2, 1)
    assert not np.any(got[dead])


# ---------------------------------------------------------------------------
# Forward: the extended-mask instances (EXT = 1 interval masks, EXT = 2 score
# modifiers), with and without a dense bias, at D = 64 and 128
# ---------------------------------------------------------------------------

EXT_CASES = [
    # D, ext kind, bias
    (128, "window", False), (128, "window", True), (128, "alibi", False), (128, "alibi", True),
    (64, "window", False), (64, "window", True), (64, "alibi", False), (64, "alibi", True),
]


def _ext_objects(kind, with_bias, B, Hq, Lq, Lk, device):
    import torch
    from probjax_amd import masks as M

    bias_np = rng_normal(62, (B, Hq, Lq, Lk), scale=0.5)[0] if with_bias else None
    if kind == "window":
        mask, omask = M.LocalWindowMask(70, 20), oracle.LocalWindowMask(70, 20)
        bias, obias = None, None
    else:
        mask, omask = M.CausalMask(), oracle.CausalMask()
        bias, obias = M.CausalAlibiBias(), oracle.CausalAlibiBias()
    if with_bias:
        db, odb = M.DenseBias(torch.from_numpy(bias_np).to(device)), oracle.DenseBias(bias_np)
        bias, obias = (db, odb) if bias is None else (bias + db, obias + odb)
    return mask, bias, omask, obias


@pytest.mark.parametrize("D,kind,with_bias", EXT_CASES)
def test_forward_extended_branch(device, D, kind, with_bias):
    import torch
    from probjax_amd import attention as A
    from probjax_amd.hip_attention import flash_attention_fwd

    B, Lq, Lk, Hq, Hkv = 2, 200, 232, 4, 2
    ext = 1 if kind == "window" else 2
    expect = f"flash_fwd_bf16_kernel<Bf16Fmt, {D}, {'true' if with_bias else 'false'}, {ext}>"
    print(f"fwd ext {kind} bias={with_bias} D={D} -> {expect}", flush=True)
    mask, bias, omask, obias = _ext_objects(kind, with_bias, B, Hq, Lq, Lk, device)
    q, k, v = (oracle.round_bf16(x) for x in rng_normal(63, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D)))
    scale = 1.0 / math.sqrt(D)
    want, want_lse = oracle.xla_attention(q, k, v, mask=omask, bias=obias, sm_scale=scale, dtype="bf16",
                                          return_lse=True)
    tq, tk, tv = (to_dev(x, device, torch.bfloat16) for x in (q, k, v))
    e = A._eligible(tq, tk, tv, mask=mask, bias=bias, dropout_rate=0.0)
    plan = A._flash_plan(tq, tk, tv, e[0], e[1])
    got, lse = flash_attention_fwd(tq, tk, tv, sm_scale=scale, return_lse=True, **plan)
    launched = _launched()
    torch.cuda.synchronize()
    assert launched == [expect], launched
    got, lse = to_np(got), to_np(lse)
    assert max_abs(got, want) <= 2e-2
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(want_lse))
    fin = np.isfinite(want_lse)
    assert max_abs(lse[fin], want_lse[fin]) <= 1e-2


# ---------------------------------------------------------------------------
# Backward: run_bwd_h16 (dQ then dK/dV), small grids (two wave groups, NG = 2)
# and large grids (NG = 1), without bias, with a dense bias, with dbias; and
# pjx_flash_bwd's D = 256 route
# ---------------------------------------------------------------------------

BWD_CASES = {
    # name: D, B, Lq, Lk, Hq, Hkv, causal, kv_lengths, bias mode, (dq NG, dkdv NG)
    "d128_large_gqa": (128, 1, 256, 256, 520, 260, True, None, None, (1, 1)),
    "d128_large_ragged": (128, 2, 256, 300, 280, 140, False, [300, 111], None, (1, 1)),
    "d128_large_bias": (128, 1, 256, 256, 520, 260, True, None, "bias", (1, 1)),
    "d128_large_dbias": (128, 2, 256, 256, 272, 272, True, [256, 200], "dbias", (1, 1)),
    "d64_large_gqa_ragged": (64, 2, 256, 256, 540, 270, True, [256, 140], None, (1, 1)),
    "d64_large_bias": (64, 1, 384, 384, 260, 260, False, None, "bias", (1, 1)),
    "d64_large_dbias": (64, 1, 256, 256, 520, 260, True, None, "dbias", (1, 1)),
    # dQ on many query tiles, dK/dV on few key blocks (GQA 8): the two branches differ
    "d128_dq_large_dkdv_small": (128, 1, 256, 256, 520, 65, True, None, None, (1, 2)),
    # small grids: both kernels in the two-group form
    "d128_small": (128, 2, 300, 300, 8, 2, True, [300, 170], None, (2, 2)),
    "d128_small_bias": (128, 1, 256, 256, 8, 8, False, None, "bias", (2, 2)),
    "d64_small_dbias": (64, 2, 200, 256, 4, 4, True, [256, 90], "dbias", (2, 2)),
    # D = 256 (two-kernel route; the dS route is tests/test_gpu_bwd_ds_route.py):
    # the wide dQ kernel, then the column-split wide dC kernel without bias,
    # the 32-key dK/dV kernel with one (no grid-size branches)
    "d256_gqa": (256, 1, 256, 256, 8, 4, True, None, None, None),
    "d256_ragged_bias": (256, 2, 200, 300, 4, 2, False, [300, 123], "bias", None),
    "d256_dbias": (256, 1, 256, 256, 4, 4, True, None, "dbias", None),
}


def _bwd_instances(E, D, mode, ng):
    dq_bias = {None: 0, "bias": 1, "dbias": 2}[mode]
    kv_bias = "false" if mode is None else "true"
    if D == 256:
        kv = f"wide_bwd_dc_kernel<{E}, 256, 256, false>" if mode is None else f"flash_bwd_dkdv_kernel<{E}, 256, true, 0, 1>"
        return [f"wide_bwd_dq_kernel<{E}, 256, 256, false, {dq_bias}, 0>", kv]
    return [f"flash_bwd_dq_kernel<{E}, {D}, {dq_bias}, 0, {ng[0]}>",
            f"flash_bwd_dkdv_kernel<{E}, {D}, {kv_bias}, 0, {ng[1]}>"]


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("name", list(BWD_CASES))
def test_backward_branch(device, name, dtype):
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    _require_256_cus()
    D, B, Lq, Lk, Hq, Hkv, causal, lengths, mode, ng = BWD_CASES[name]
    expect = _bwd_instances(FMT[dtype], D, mode, ng)
    print(f"bwd {name} {dtype}: D={D} B={B} Lq={Lq} Lk={Lk} Hq={Hq} Hkv={Hkv} causal={causal} "
          f"lengths={lengths} bias={mode} -> {expect}", flush=True)
    q, k, v, do = (_round(x, dtype) for x in rng_normal(64, (B, Lq, Hq, D), (B, Lk, Hkv, D), (B, Lk, Hkv, D),
                                                        (B, Lq, Hq, D)))
    bias = None if mode is None else rng_normal(65, (1, Hq, Lq, Lk), scale=0.5)[0]
    scale = 1.0 / math.sqrt(D)
    mask = _omask(causal, lengths, Lk)
    db = None if bias is None else oracle.DenseBias(bias)
    o, lse = oracle.xla_attention(q, k, v, mask=mask, bias=db, sm_scale=scale, dtype=dtype,
                                  return_lse=True)
    want = attention_backward(q, k, v, o, do, lse, mask=mask, bias=db, sm_scale=scale, dtype=dtype,
                              return_dbias=mode == "dbias")
    tdt = _tdt(dtype)
    L = None if lengths is None else torch.tensor(lengths, dtype=torch.int32, device=device)
    bt = None if bias is None else torch.from_numpy(bias).to(device)
    got = flash_attention_bwd(
        to_dev(q, device, tdt), to_dev(k, device, tdt), to_dev(v, device, tdt), to_dev(o, device, tdt),
        to_dev(do, device, tdt), torch.from_numpy(lse).to(device), sm_scale=scale, causal=causal,
        kv_lengths=L, bias=bt, bias_grad=mode == "dbias", ds_route=False,
    )
    launched = _launched()
    torch.cuda.synchronize()
    assert launched == expect, launched
    names = ("dq", "dk", "dv", "dbias")
    if mode == "dbias":
        want = (*want[:3], want[3].sum(axis=0, keepdims=True))  # bias [1, Hq, Lq, Lk]
    for nm, g, w in zip(names, got, want):
        _check_grad(to_np(g), w, nm)
    if lengths is not None:
        for b, n in enumerate(lengths):
            assert torch.count_nonzero(got[1][b, n:]) == 0 and torch.count_nonzero(got[2][b, n:]) == 0
