"""Benchmark of the MI355X fused-attention path (one GPU).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Headline workload (the BASELINE metric's prefill half): the bf16 causal flash
forward at B=4, H=16, L=4096, D=128 (``configs[1]``).  One step = one
``pjx_flash_fwd`` call over that batch, inputs resident in HBM.  ``value`` is
TFLOP/s with the reference's FLOP convention ``4*B*H*Lq*Lk*D``, halved for
causal (probjax docs/scripts/benchmark_gpu_attention.py:179-187).

Each workload first runs untimed for ``--settle`` seconds (default 0.5) so that
the GPU clocks reach their sustained level, then W warmup steps, then the K
timed steps.

The other configurations are measured the same way after the headline and
reported under ``"configs"`` (decode and MLA as HBM GB/s of the bytes the
algorithm must move: valid K/V + q + o; bias configs include the bias once).
``C2B`` is the backward of the headline workload (one ``pjx_flash_bwd`` call)
and ``C2FB`` forward + backward, both as TFLOP/s with the reference
benchmark's FlashAttention convention (fwd+bwd = 3.5x the forward's FLOPs).
``C5P`` is the materialised-MLA up-projection alone (``pjx_mla_project``) and
``C5M`` a materialised-MLA causal prefill (projection + flash forward).
``C5A`` is the absorbed-MLA causal prefill (``pjx_mla_fwd``, B=1, L=4096,
H=16, R=576, 512 value columns) and ``C5AB`` its backward (``pjx_mla_bwd``);
``C2W`` a head-dim-256 causal forward.

``cpu_baseline`` times the numpy restatement of probjax's XLA CPU path
(``oracle.xla_attention``, 256x256 tiles with causal tile skipping) on one
(batch, head) slice of the headline workload on the host cores, and scales it
to TFLOP/s; its ``decode`` entry times the same path on the first 4 of C3's
32 sequences, as GB/s of the bytes that slice must read.  Both are reported
baselines only.

``--summarize-trace DIR`` prints, per workload, the kernels of the timed
steps of a ``rocprofv3 --kernel-trace --marker-trace`` run of this script
(each workload's timed steps sit in a roctx range).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3     # MI355X fp32 matrix
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

METRIC = "flash-attn fwd TFLOP/s (% bf16 MFMA peak); split-KV decode HBM GB/s (% peak)"


def _parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--settle", type=float, default=0.5, metavar="SECONDS",
                   help="untimed clock-settling run of each workload before its warmup steps")
    p.add_argument("--no-cpu-baseline", action="store_true",
                   help="skip the timed CPU oracle leg")
    p.add_argument("--only", default="",
                   help="comma list of configs to run (C1..C5, C2B = backward, C2FB = "
                        "forward+backward); default all")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="only run a plain device copy of MIB MiB (counter calibration) and exit")
    p.add_argument("--summarize-trace", default="", metavar="DIR",
                   help="only summarise a rocprofv3 --kernel-trace --marker-trace csv run of this script "
                        "(the kernels of each workload's timed steps) and exit; needs no GPU")
    p.add_argument("--gemm-calibration", type=int, default=0, metavar="N",
                   help="only time a library bf16 GEMM N x N x N (torch.matmul -> hipBLASLt), the "
                        "practical MFMA ceiling on this box, and exit")
    return p.parse_args()


def copy_calibration(mib, reps=5):
    """A plain device-to-device copy of known size: the reference point that
    scales FETCH_SIZE / WRITE_SIZE counter readings to bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_each_way": n * 4, "reps": reps}), flush=True)


def gemm_calibration(n, settle_s, steps=10):
    """A library bf16 GEMM (torch.matmul, hipBLASLt) after clock settling:
    the MFMA rate a plain GEMM sustains within this box's power limit."""
    import torch

    a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16)
    fn = lambda: torch.matmul(a, b)  # noqa: E731
    wall_ms, ev_ms = _time(fn, steps, 2, settle_s)
    print(json.dumps({"gemm_calibration": f"bf16 {n}x{n}x{n}", "ms": round(ev_ms, 4),
                      "tflops": round(2 * n ** 3 / (ev_ms * 1e-3) / 1e12, 1)}), flush=True)


# ---------------------------------------------------------------------------
# Workloads: each returns (name, fn, flop, bytes, bound, dtype, extra dict)
# ---------------------------------------------------------------------------

def _randn(shape, gen, dev, dtype, scale=1.0):
    import torch

    x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


def make_c1(dev, gen):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 1, 512, 4, 64
    q, k, v = (_randn((B, L, H, D), gen, dev, torch.float32) for _ in range(3))
    flop = 4 * B * H * L * L * D / 2
    nbytes = 4 * B * L * H * D * 4
    fn = lambda: flash_attention_fwd(q, k, v, sm_scale=1 / 8, causal=True)  # noqa: E731
    return dict(name="C1 causal fwd f32 B=1 H=4 L=512 D=64", fn=fn, flop=flop, bytes=nbytes,
                bound="latency", dtype="f32", kernel="flash_fwd_f32_split_kernel<64,false>")


def make_c2(dev, gen):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 4, 4096, 16, 128
    q, k, v = (_randn((B, L, H, D), gen, dev, torch.bfloat16) for _ in range(3))
    flop = 4 * B * H * L * L * D / 2
    nbytes = 4 * B * L * H * D * 2
    fn = lambda: flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True)  # noqa: E731
    return dict(name="C2 causal fwd bf16 B=4 H=16 L=4096 D=128", fn=fn, flop=flop, bytes=nbytes,
                bound="mfma", dtype="bf16", kernel="flash_fwd_bf16_pipe_kernel<Bf16Fmt,128,32,3,1>")


def make_c2h(dev, gen):
    """C2 in float16 (the same kernel on v_mfma_f32_32x32x16_f16)."""
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 4, 4096, 16, 128
    q, k, v = (_randn((B, L, H, D), gen, dev, torch.float16) for _ in range(3))
    flop = 4 * B * H * L * L * D / 2
    nbytes = 4 * B * L * H * D * 2
    fn = lambda: flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True)  # noqa: E731
    return dict(name="C2 causal fwd fp16 B=4 H=16 L=4096 D=128", fn=fn, flop=flop, bytes=nbytes,
                bound="mfma", dtype="f16", kernel="flash_fwd_bf16_pipe_kernel<F16Fmt,128,32,3,1>")


def c3_lengths(seed=0, batch=32, lo=512, hi=8192):
    """Per-sequence valid lengths, uniform integers in [lo, hi] (seeded)."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=batch).astype(np.int32)


def make_c3(dev, gen):
    import torch
    from probjax_amd.hip_attention import decode_workspace_bytes, splitkv_decode

    B, S, Hq, Hkv, D = 32, 8192, 32, 8, 128
    q = _randn((B, 1, Hq, D), gen, dev, torch.bfloat16)
    k = _randn((B, S, Hkv, D), gen, dev, torch.bfloat16)
    v = _randn((B, S, Hkv, D), gen, dev, torch.bfloat16)
    lens = c3_lengths()
    L = torch.from_numpy(lens).to(dev)
    ws = torch.empty(decode_workspace_bytes(B, Hkv, Hq // Hkv, S, D), dtype=torch.uint8, device=dev)
    tot = int(lens.sum())
    nbytes = tot * Hkv * D * 2 * 2 + 2 * B * Hq * D * 2
    flop = 4 * Hq * D * tot
    fn = lambda: splitkv_decode(q, k, v, sm_scale=1 / math.sqrt(D), kv_lengths=L, workspace=ws)  # noqa: E731
    return dict(name="C3 GQA split-KV decode bf16 B=32 Hq=32 Hkv=8 D=128 S=8192 ragged",
                fn=fn, flop=flop, bytes=nbytes, bound="hbm", dtype="bf16",
                kernel="gqa_decode_kernel<Bf16Fmt, 128, 128, 1, true> + decode_merge_kernel", sum_len=tot)


def c4_lengths(seed=0, batch=2, length=2048):
    """Valid keys per sequence: the last ~10% dropped, offset jittered by +-16 (seeded)."""
    rng = np.random.default_rng(seed)
    drop = int(round(0.1 * length)) + rng.integers(-16, 17, size=batch)
    return (length - drop).astype(np.int32)


def make_c4(dev, gen):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 2, 2048, 8, 64
    q, k, v = (_randn((B, L, H, D), gen, dev, torch.bfloat16) for _ in range(3))
    bias = _randn((1, H, L, L), gen, dev, torch.float32, scale=0.5)
    L_ = torch.from_numpy(c4_lengths()).to(dev)
    flop = 4 * B * H * L * L * D
    nbytes = H * L * L * 4 + 4 * B * L * H * D * 2
    fn = lambda: flash_attention_fwd(q, k, v, sm_scale=1 / 8, kv_lengths=L_, bias=bias)  # noqa: E731
    return dict(name="C4 bias+kvlen fwd bf16 B=2 H=8 L=2048 D=64, bias f32 [8,2048,2048]",
                fn=fn, flop=flop, bytes=nbytes, bound="hbm", dtype="bf16",
                kernel="flash_fwd_bf16_bias_ring_kernel<Bf16Fmt,64,3>")


def make_c5(dev, gen):
    import torch
    from probjax_amd.hip_attention import decode_workspace_bytes, mla_decode

    B, H, S, R, DV = 16, 16, 4096, 576, 512
    q = _randn((B, 1, H, R), gen, dev, torch.bfloat16)
    cache = _randn((B, S, R), gen, dev, torch.bfloat16)
    ws = torch.empty(decode_workspace_bytes(B, 1, H, S, DV), dtype=torch.uint8, device=dev)
    nbytes = B * S * R * 2 + B * H * R * 2 + B * H * R * 2
    flop = 2 * B * H * S * (R + DV)
    fn = lambda: mla_decode(q, cache, sm_scale=1 / math.sqrt(192), v_dim=DV, workspace=ws)  # noqa: E731
    return dict(name="C5 MLA absorbed decode bf16 B=16 H=16 S=4096 R=576 Dv=512",
                fn=fn, flop=flop, bytes=nbytes, bound="hbm", dtype="bf16",
                kernel="mla_decode_kernel<Bf16Fmt, 576, 512, false> + decode_merge_kernel")


def _c2_train_inputs(dev, gen):
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 4, 4096, 16, 128
    q, k, v, do = (_randn((B, L, H, D), gen, dev, torch.bfloat16) for _ in range(4))
    o, lse = flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True, return_lse=True)
    return B, L, H, D, q, k, v, do, o, lse


def make_c2b(dev, gen):
    """Backward of the headline forward: one pjx_flash_bwd call (dq, dk, dv).

    FLOPs by the FlashAttention convention of the reference's benchmark
    (docs/scripts/benchmark_gpu_attention.py:179-187: fwd+bwd = 3.5x fwd, so
    bwd = 2.5x fwd); the kernels execute 3.5x fwd (S and dP are recomputed
    for dQ)."""
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd

    B, L, H, D, q, k, v, do, o, lse = _c2_train_inputs(dev, gen)
    ws = torch.empty(8 * B * H * L, dtype=torch.uint8, device=dev)
    flop = 2.5 * 4 * B * H * L * L * D / 2
    nbytes = 2 * B * L * H * D * 2 * 4 + B * H * L * 4  # q,k,v,o,do + dq,dk,dv + lse
    fn = lambda: flash_attention_bwd(q, k, v, o, do, lse, sm_scale=1 / math.sqrt(D), causal=True,  # noqa: E731
                                     workspace=ws)
    return dict(name="C2 causal bwd bf16 B=4 H=16 L=4096 D=128 (dq, dk, dv)", fn=fn, flop=flop,
                bytes=nbytes, bound="mfma", dtype="bf16",
                kernel="flash_bwd_dq_kernel<Bf16Fmt,128,0,0,1> + flash_bwd_dkdv_kernel<Bf16Fmt,128,false,0,1>")


def make_c2fb(dev, gen):
    """Forward (with LSE) + backward, the reference benchmark's fwd_bwd mode
    (3.5x the forward's FLOPs)."""
    import torch
    from probjax_amd.hip_attention import flash_attention_bwd, flash_attention_fwd

    B, L, H, D, q, k, v, do, _, _ = _c2_train_inputs(dev, gen)
    ws = torch.empty(8 * B * H * L, dtype=torch.uint8, device=dev)
    sc = 1 / math.sqrt(D)

    def fn():
        o, lse = flash_attention_fwd(q, k, v, sm_scale=sc, causal=True, return_lse=True)
        return flash_attention_bwd(q, k, v, o, do, lse, sm_scale=sc, causal=True, workspace=ws)

    flop = 3.5 * 4 * B * H * L * L * D / 2
    nbytes = 2 * B * L * H * D * 2 * 5 + B * H * L * 4
    return dict(name="C2 causal fwd+bwd bf16 B=4 H=16 L=4096 D=128", fn=fn, flop=flop,
                bytes=nbytes, bound="mfma", dtype="bf16",
                kernel="flash_fwd_bf16_pipe_kernel<Bf16Fmt,128,32,3,1> + flash_bwd_dq_kernel<Bf16Fmt,128,0,0,1> + flash_bwd_dkdv_kernel<Bf16Fmt,128,false,0,1>")


def _mla_prefill_inputs(dev, gen):
    import torch

    B, L, H, R, D = 1, 4096, 16, 512, 128
    q = _randn((B, L, H, D), gen, dev, torch.bfloat16)
    cache = _randn((B, L, R), gen, dev, torch.bfloat16)
    wk, wv = (_randn((H, D, R), gen, dev, torch.bfloat16, scale=1 / math.sqrt(R)) for _ in range(2))
    return B, L, H, R, D, q, cache, wk, wv


def make_c5p(dev, gen):
    """The latent up-projection alone (pjx_mla_project: K and V of a 4096-token
    latent, 16 heads x 128), a GEMM of 2 * M * R * N FLOPs."""
    from probjax_amd.hip_attention import mla_project

    B, L, H, R, D, _, cache, wk, wv = _mla_prefill_inputs(dev, gen)
    flop = 2 * B * L * R * H * 2 * D
    nbytes = B * L * R * 2 + 2 * H * D * R * 2 + 2 * B * L * H * D * 2
    fn = lambda: mla_project(cache, wk, wv, width=D)  # noqa: E731
    return dict(name="MLA up-projection bf16 B=1 S=4096 R=512 H=16 dk=dv=128 (K and V)", fn=fn,
                flop=flop, bytes=nbytes, bound="mfma", dtype="bf16", kernel="mla_project_bf16_kernel<Bf16Fmt>")


def make_c5m(dev, gen):
    """Materialised latent attention prefill (mla with wk / wv, causal): the
    up-projection then the flash forward over the materialised K / V.  FLOPs:
    the projection's plus the causal attention's (reference convention)."""
    from probjax_amd.hip_attention import flash_attention_fwd, mla_project

    B, L, H, R, D, q, cache, wk, wv = _mla_prefill_inputs(dev, gen)
    sc = 1 / math.sqrt(D)

    def fn():
        k, v = mla_project(cache, wk, wv, width=D)
        return flash_attention_fwd(q, k, v, sm_scale=sc, causal=True)

    flop = 2 * B * L * R * H * 2 * D + 4 * B * H * L * L * D / 2
    nbytes = B * L * R * 2 + 2 * H * D * R * 2 + 2 * B * L * H * D * 2
    return dict(name="MLA materialised causal prefill bf16 B=1 L=4096 R=512 H=16 dk=dv=128", fn=fn,
                flop=flop, bytes=nbytes, bound="mfma", dtype="bf16",
                kernel="mla_project_bf16_kernel<Bf16Fmt> + flash_fwd_bf16_pipe_kernel<Bf16Fmt,128,64,2,2>")


def _latent_prefill_inputs(dev, gen):
    import torch

    B, L, H, R, DV = 1, 4096, 16, 576, 512
    q = _randn((B, L, H, R), gen, dev, torch.bfloat16)
    cache = _randn((B, L, R), gen, dev, torch.bfloat16)
    return B, L, H, R, DV, q, cache


def make_c5a(dev, gen):
    """Absorbed latent attention, causal prefill (mla(q, cache, mask=CausalMask())
    sliced to the 512 value columns, as the config-5 harness uses it):
    pjx_mla_fwd.  FLOPs by the reference convention, 2 * (R + DV) per
    (query row, head, visible key): the scores over the 576-wide latent and
    P.V over its first 512 columns; the kernel forms each score twice (once per
    256-column half of the output), which is not counted."""
    from probjax_amd.hip_attention import mla_fwd

    B, L, H, R, DV, q, cache = _latent_prefill_inputs(dev, gen)
    flop = 2 * B * H * L * L / 2 * (R + DV)
    nbytes = B * L * H * R * 2 + B * L * R * 2 + B * L * H * DV * 2
    fn = lambda: mla_fwd(q, cache, sm_scale=1 / math.sqrt(192), v_dim=DV, causal=True)  # noqa: E731
    return dict(name="MLA absorbed causal prefill bf16 B=1 L=4096 H=16 R=576 Dv=512", fn=fn, flop=flop,
                bytes=nbytes, bound="mfma", dtype="bf16", kernel="flash_fwd_wide_kernel<Bf16Fmt,576,256,32,true,false,0>")


def make_c5ab(dev, gen):
    """Backward of C5A (pjx_mla_bwd: dq and the cache gradient).  FLOPs: the
    five products per visible (row, key) pair -- scores (R) and dP (DV)
    recomputed, dQ (R), dK (R), dV (DV) -- at 2 FLOPs per multiply-add."""
    import torch
    from probjax_amd.hip_attention import mla_bwd, mla_fwd

    B, L, H, R, DV, q, cache = _latent_prefill_inputs(dev, gen)
    sc = 1 / math.sqrt(192)
    o, lse = mla_fwd(q, cache, sm_scale=sc, v_dim=DV, causal=True, return_lse=True)
    do = _randn(tuple(o.shape), gen, dev, torch.bfloat16)
    flop = 2 * B * H * L * L / 2 * (3 * R + 2 * DV)
    nbytes = 2 * B * L * H * R * 2 + 2 * B * L * R * 2 + 2 * B * L * H * DV * 2
    fn = lambda: mla_bwd(q, cache, o, do, lse, sm_scale=sc, causal=True)  # noqa: E731
    return dict(name="MLA absorbed causal prefill backward bf16 B=1 L=4096 H=16 R=576 Dv=512 (dq, dcache)",
                fn=fn, flop=flop, bytes=nbytes, bound="mfma", dtype="bf16",
                kernel="wide_bwd_dq_kernel<Bf16Fmt,576,512,true,0,0> + wide_bwd_dc_kernel<Bf16Fmt,576,512,true> + wide_bwd_reduce_kernel<Bf16Fmt>")


def make_c2w(dev, gen):
    """Head dim 256 causal flash forward (the widest head the reference's fused
    route takes), B=2, H=16, L=4096."""
    import torch
    from probjax_amd.hip_attention import flash_attention_fwd

    B, L, H, D = 2, 4096, 16, 256
    q, k, v = (_randn((B, L, H, D), gen, dev, torch.bfloat16) for _ in range(3))
    flop = 4 * B * H * L * L * D / 2
    nbytes = 4 * B * L * H * D * 2
    fn = lambda: flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(D), causal=True)  # noqa: E731
    return dict(name="causal fwd bf16 B=2 H=16 L=4096 D=256", fn=fn, flop=flop, bytes=nbytes,
                bound="mfma", dtype="bf16", kernel="flash_fwd_wide_kernel<Bf16Fmt,256,256,32,false,false,0>")


def make_c2wb(dev, gen):
    """Backward of the head-dim-256 forward (the C2W shape): one pjx_flash_bwd
    call on its dS route (the workspace holds the rounded dS: delta, the
    column-split dK/dV kernel storing dS, then dQ = dS K).  FLOPs by the
    2.5x-forward convention, as for C2B."""
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import flash_attention_bwd, flash_attention_fwd

    B, L, H, D = 2, 4096, 16, 256
    q, k, v, do = (_randn((B, L, H, D), gen, dev, torch.bfloat16) for _ in range(4))
    sc = 1 / math.sqrt(D)
    o, lse = flash_attention_fwd(q, k, v, sm_scale=sc, causal=True, return_lse=True)
    nws = int(native.load().pjx_flash_bwd_ds_workspace_size(native.PJX_DTYPE_BF16, B, H, L, L, D))
    ws = torch.empty(nws, dtype=torch.uint8, device=dev)
    flop = 2.5 * 4 * B * H * L * L * D / 2
    nbytes = 2 * B * L * H * D * 2 * 4 + B * H * L * 4
    fn = lambda: flash_attention_bwd(q, k, v, o, do, lse, sm_scale=sc, causal=True, workspace=ws)  # noqa: E731
    return dict(name="causal bwd bf16 B=2 H=16 L=4096 D=256 (dq, dk, dv)", fn=fn, flop=flop, bytes=nbytes,
                bound="mfma", dtype="bf16",
                kernel="wide_bwd_delta_kernel<Bf16Fmt,256> + wide_bwd_dc_ds_kernel<Bf16Fmt,256,256,false> + "
                       "wide_bwd_dq_ds_kernel<Bf16Fmt,256>")


MAKERS = {"C1": make_c1, "C2": make_c2, "C3": make_c3, "C4": make_c4, "C5": make_c5,
          "C2B": make_c2b, "C2FB": make_c2fb, "C5P": make_c5p, "C5M": make_c5m,
          "C5A": make_c5a, "C5AB": make_c5ab, "C2W": make_c2w, "C2H": make_c2h, "C2WB": make_c2wb}


def _settle(fn, seconds):
    """Untimed clock settling: run the workload for `seconds` of wall time.

    MI355X raises its clocks over the first tens of milliseconds of sustained
    load; a C2 step measured after 5 warmup calls reads ~25% slower than
    after 200.  Settling before the W warmup steps makes the K timed steps
    the steady state whatever W the caller passes."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


TIMED_RANGE = "pjx-timed:"  # roctx range name prefix around each workload's timed steps


def _time(fn, steps, warmup, settle_s=0.0, label=None):
    """Wall time of `steps` back-to-back calls between device syncs, and the
    per-call average from HIP events recorded on the launch stream.  With a
    label, the timed steps (and nothing else) sit in a roctx range
    ``pjx-timed:<label>``, so a ``rocprofv3 --kernel-trace --marker-trace``
    run can quote the kernels of exactly those steps (``--summarize-trace``)."""
    import torch

    _settle(fn, settle_s)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    if label is not None:
        torch.cuda.nvtx.range_push(TIMED_RANGE + label)
    stream = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if label is not None:
        torch.cuda.nvtx.range_pop()
    return wall / steps * 1e3, e0.elapsed_time(e1) / steps


def summarize_trace(trace_dir):
    """Per workload, the kernels dispatched inside its timed range in a
    ``rocprofv3 --kernel-trace --marker-trace --output-format csv`` run of this
    script (``*_kernel_trace.csv``, ``*_marker_api_trace.csv`` in trace_dir):
    calls, average / min / max duration, and the workload's kernel time per
    step (sum of durations / steps).  Prints a markdown table."""
    import csv
    import glob
    import re

    def one(pattern):
        files = glob.glob(os.path.join(trace_dir, "**", pattern), recursive=True)
        if len(files) != 1:
            raise SystemExit(f"--summarize-trace: expected one {pattern} under {trace_dir}, found {files}")
        with open(files[0]) as f:
            return list(csv.DictReader(f))

    ranges = [(r["Function"][len(TIMED_RANGE):], int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
              for r in one("*marker_api_trace.csv") if r["Function"].startswith(TIMED_RANGE)]
    def short(name):
        return re.sub(r"^void |\(.*$", "", name.replace("(anonymous namespace)::", ""))

    kernels = [(short(r["Kernel_Name"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
               for r in one("*kernel_trace.csv")]
    print("| workload | kernel | calls | avg µs | min µs | max µs | kernel µs per step |")
    print("|---|---|---|---|---|---|---|")
    for label, t0, t1 in ranges:
        per = {}
        for name, k0, k1 in kernels:
            if k0 >= t0 and k1 <= t1:
                per.setdefault(name, []).append((k1 - k0) / 1e3)
        steps = max((len(v) for v in per.values()), default=1)
        for name, d in sorted(per.items(), key=lambda kv: -sum(kv[1])):
            print(f"| {label} | `{name}` | {len(d)} | {sum(d) / len(d):.1f} | {min(d):.1f} | {max(d):.1f} | "
                  f"{sum(d) / steps:.1f} |")


def _rates(w, ms):
    tflops = w["flop"] / (ms * 1e-3) / 1e12
    gbs = w["bytes"] / (ms * 1e-3) / 1e9
    if w["bound"] == "hbm":
        frac = gbs / PEAK_HBM_GBS
    elif w["dtype"] == "f32":
        frac = tflops / PEAK_F32_TFLOPS
    else:
        frac = tflops / PEAK_BF16_TFLOPS
    return tflops, gbs, frac


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_bench.json")


def measured_traffic(kernel_key):
    """HBM bytes per launch of a kernel from the committed rocprofv3 counter
    summary (FETCH_SIZE + WRITE_SIZE, each scaled by the plain-copy
    calibration), or None when the summary does not cover it."""
    try:
        with open(TRAFFIC_FILE) as f:
            table = json.load(f)
    except (OSError, ValueError):
        return None
    row = table.get("kernels", {}).get(kernel_key)
    return None if not row or row.get("hbm_bytes") is None else int(row["hbm_bytes"])


def cpu_baseline(target_s=10.0):
    """numpy XLA-path restatement on one (b, h) slice of the headline workload."""
    import oracle

    threads = len(os.sched_getaffinity(0))
    try:
        from threadpoolctl import threadpool_limits

        limiter = threadpool_limits(limits=threads)
    except Exception:  # pragma: no cover - threadpoolctl is optional
        limiter = None
    rng = np.random.default_rng(0)
    L, D = 4096, 128
    q, k, v = (oracle.round_bf16(rng.standard_normal((1, L, 1, D), dtype=np.float32))
               for _ in range(3))
    flop = 4 * L * L * D / 2
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.xla_attention(q, k, v, mask=oracle.CausalMask(), sm_scale=1 / math.sqrt(D),
                             dtype="bf16")
        n += 1
        el = time.perf_counter() - t0
        if el >= target_s or n >= 1000:
            break
    per = el / n
    out = {
        "value": flop / per / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": f"numpy restatement of xla_attention (256x256 tiles, causal tile skip, bf16 P "
                  f"rounding), one (b,h) slice 1x4096x1x128 of C2, {n} runs, {per * 1e3:.1f} ms each",
    }
    # the decode half of the metric: a slice of C3 (its first sequences, the
    # same seeded lengths), GB/s of the valid K/V rows + q + o it must read
    nb, S, Hq, Hkv, D = 4, 8192, 32, 8, 128
    lens = c3_lengths()[:nb]
    q = oracle.round_bf16(rng.standard_normal((nb, 1, Hq, D), dtype=np.float32))
    k, v = (oracle.round_bf16(rng.standard_normal((nb, S, Hkv, D), dtype=np.float32)) for _ in range(2))
    nbytes = int(lens.sum()) * Hkv * D * 2 * 2 + 2 * nb * Hq * D * 2
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.xla_attention(q, k, v, mask=oracle.KVLenMask(lens), sm_scale=1 / math.sqrt(D), dtype="bf16")
        n += 1
        el = time.perf_counter() - t0
        if el >= target_s / 2 or n >= 1000:
            break
    if limiter is not None:
        limiter.unregister() if hasattr(limiter, "unregister") else None
    per = el / n
    out["decode"] = {
        "value": nbytes / per / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"numpy restatement of xla_attention with KVLenMask, bf16 P rounding: the first {nb} "
                  f"of C3's 32 sequences (lengths {lens.tolist()}, Hq=32 over Hkv=8, D=128, capacity "
                  f"{S}), {n} runs, {per * 1e3:.1f} ms each; GB/s of the valid K/V rows + q + o",
    }
    return out


def main():
    args = _parse()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "the path's multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        sys.exit(1)
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gemm_calibration:
        gemm_calibration(args.gemm_calibration, args.settle)
        return
    from probjax_amd import native

    native.load()
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    only = [s.strip() for s in args.only.split(",") if s.strip()] or list(MAKERS)

    results = {}
    head = None
    for key in only:
        w = MAKERS[key](dev, gen)
        wall_ms, ev_ms = _time(w["fn"], args.steps, args.warmup, args.settle, label=key)
        tflops, gbs, frac = _rates(w, ev_ms)
        row = {"workload": w["name"], "ms": round(ev_ms, 5), "wall_ms": round(wall_ms, 5),
               "tflops": round(tflops, 2), "gbs": round(gbs, 1),
               "roofline_bound": w["bound"], "roofline_frac": round(frac, 4),
               "dtype": w["dtype"]}
        if "sum_len" in w:
            row["sum_valid_len"] = w["sum_len"]
        results[key] = row
        print(f"[bench] {key}: {json.dumps(row)}", file=sys.stderr, flush=True)
        if key == "C2":
            head = (w, wall_ms, ev_ms, tflops, frac)
        del w
        torch.cuda.empty_cache()

    out = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "settle_s": args.settle,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "data": "synthetic (torch.randn N(0,1) on device, seed 0)"}
    if head is not None:
        w, wall_ms, ev_ms, tflops, frac = head
        out.update({
            "value": round(w["flop"] / (wall_ms * 1e-3) / 1e12, 2),
            "unit": "TFLOP/s",
            "ms_per_step": round(wall_ms, 5),
            "dtype": "bf16",
            "config": {"workload": w["name"], "batch": 4, "heads": 16, "seq_len": 4096,
                       "head_dim": 128, "mask": "causal", "flop_per_step": w["flop"]},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(frac, 4),
                         "traffic": measured_traffic("pjx::flash_fwd_bf16_pipe_kernel<pjx::Bf16Fmt, 128, 32, 3, 1>"),
                         "traffic_unit": "bytes per launch (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
                         "kernel": w["kernel"]},
        })
    if "C3" in results:
        r = results["C3"]
        out["decode_roofline"] = {"bound": "hbm", "achieved": r["gbs"], "peak": PEAK_HBM_GBS,
                                  "unit": "GB/s", "frac": r["roofline_frac"],
                                  "traffic": measured_traffic("pjx::gqa_decode_kernel<pjx::Bf16Fmt, 128, 128, 1, true>"),
                                  "kernel": "gqa_decode_kernel<Bf16Fmt, 128, 128, 1, true> + decode_merge_kernel"}
    out["configs"] = results
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
