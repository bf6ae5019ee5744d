"""The kernels under HIP graph capture and under concurrent callers.

* A captured step (flash forward and backward, split-KV decode with a caller
  workspace, the no-allocation decode, the latent decode) replayed several
  times, with new inputs written in place and unrelated eager work between
  replays, must give what eager calls give on the same inputs, bitwise.  The
  library records no memset into a graph (zero fills are kernels), and its
  launches take the capturing stream.
* Several host threads on their own streams at once (the boundary's
  contract: handlers are stateless and reentrant) give what one thread gives.
"""

import ctypes
import math

import pytest

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(device):
    import torch
    from probjax_amd import native
    from probjax_amd.hip_attention import (decode_workspace_bytes, flash_attention_bwd, flash_attention_fwd,
                                           mla_decode, splitkv_decode)

    lib = native.load()
    g = torch.Generator(device=device)
    g.manual_seed(81)
    bf = torch.bfloat16

    def rnd(*shape):
        return torch.randn(shape, generator=g, device=device).to(bf)

    # static inputs, refilled in place before every replay
    q, do = rnd(2, 300, 4, 128), rnd(2, 300, 4, 128)
    k, v = rnd(2, 300, 2, 128), rnd(2, 300, 2, 128)
    qd, kd, vd = rnd(3, 1, 8, 128), rnd(3, 1500, 2, 128), rnd(3, 1500, 2, 128)
    Ld = torch.tensor([1500, 700, 0], dtype=torch.int32, device=device)
    qm, cm = rnd(2, 1, 16, 576), rnd(2, 900, 576)
    Lm = torch.tensor([900, 333], dtype=torch.int32, device=device)
    ws_d = torch.empty(decode_workspace_bytes(3, 2, 4, 1500, 128), dtype=torch.uint8, device=device)
    ws_m = torch.empty(decode_workspace_bytes(2, 1, 16, 900, 512), dtype=torch.uint8, device=device)
    inputs = (q, do, k, v, qd, kd, vd, qm, cm)

    def step():
        o, lse = flash_attention_fwd(q, k, v, sm_scale=1 / math.sqrt(128), causal=True, return_lse=True)
        dq, dk, dv = flash_attention_bwd(q, k, v, o, do, lse, sm_scale=1 / math.sqrt(128), causal=True)
        od = splitkv_decode(qd, kd, vd, sm_scale=0.1, kv_lengths=Ld, workspace=ws_d)
        os_ = torch.empty_like(od)
        stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
        native.check(lib.pjx_splitkv_decode_static(
            native.PJX_DTYPE_BF16, *(ctypes.c_void_p(t.data_ptr()) for t in (qd, kd, vd, Ld, os_)), None,
            3, 1, 1500, 8, 2, 128, 128, ctypes.c_float(0.1), 0, stream))
        om = mla_decode(qm, cm, sm_scale=1 / math.sqrt(192), v_dim=512, kv_lengths=Lm, workspace=ws_m)
        return [o, lse, dq, dk, dv, od, os_, om]

    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        step()   # warm-up off the default stream, as torch's capture recipe asks
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for rep in range(4):
        print(f"graph replay {rep}", flush=True)
        for t in inputs:
            t.copy_(torch.randn(t.shape, generator=g, device=device).to(bf))
        x = torch.randn((512, 512), generator=g, device=device)
        (x @ x).sum().item()   # unrelated eager work and a host sync between replays
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in captured]
        want = step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a, b), f"replay {rep}, output {i}"


def test_concurrent_host_threads_and_streams(device):
    """The entry points keep no state between calls (error text and launch log
    are per host thread): four host threads, each on its own stream, running
    the forward, backward and split-KV decode on their own inputs at the same
    time give what one thread gives on the same inputs, bitwise."""
    import threading

    import torch
    from probjax_amd.hip_attention import flash_attention_bwd, flash_attention_fwd, splitkv_decode

    g = torch.Generator(device=device)
    g.manual_seed(91)
    bf = torch.bfloat16

    def make(i):
        r = lambda *s: torch.randn(s, generator=g, device=device).to(bf)  # noqa: E731
        return dict(q=r(1, 512 + 64 * i, 4, 128), k=r(1, 512 + 64 * i, 2, 128), v=r(1, 512 + 64 * i, 2, 128),
                    do=r(1, 512 + 64 * i, 4, 128), qd=r(2, 1, 8, 64), kd=r(2, 3000, 1, 64), vd=r(2, 3000, 1, 64),
                    L=torch.tensor([3000, 1111 * (i + 1)], dtype=torch.int32, device=device))

    def work(x):
        o, lse = flash_attention_fwd(x["q"], x["k"], x["v"], sm_scale=0.09, causal=True, return_lse=True)
        dq, dk, dv = flash_attention_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, sm_scale=0.09, causal=True)
        od = splitkv_decode(x["qd"], x["kd"], x["vd"], sm_scale=0.12, kv_lengths=x["L"])
        return [o, lse, dq, dk, dv, od]

    inputs = [make(i) for i in range(4)]
    want = [work(x) for x in inputs]
    torch.cuda.synchronize()
    got = [None] * 4
    errors = []

    def run(i):
        try:
            s = torch.cuda.Stream(device)
            with torch.cuda.stream(s):
                for _ in range(3):
                    res = work(inputs[i])
                s.synchronize()
            got[i] = res
        except Exception as e:  # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(4):
        for j, (a, b) in enumerate(zip(got[i], want[i])):
            assert torch.equal(a, b), f"thread {i}, output {j}"
