"""The C-ABI library loads and exports every entry point its header declares.

No kernel is launched here: only argument validation paths that return
before any HIP call are exercised, so this runs without a GPU.
"""

import ctypes
import re
from pathlib import Path

import pytest

from probjax_amd import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "probjax_hip.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pjx_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not native.LIB_PATH.exists():
        pytest.fail(f"{native.LIB_PATH} is not built: run __graft_entry__.build()")
    return native.load()


def test_header_declarations_are_bound():
    declared = _declared()
    assert declared, "no entry points parsed from the header"
    assert sorted(native.EXPORTED) == declared


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert getattr(lib, name, None) is not None, name


def test_version_and_error_string(lib):
    assert lib.pjx_version() >= 100
    assert isinstance(lib.pjx_last_error(), bytes)


def _flash_args(**over):
    a = dict(dtype=native.PJX_DTYPE_BF16, q=1, k=1, v=1, o=1, lse=None, kvl=None, bias=None,
             bb=1, bh=1, B=1, Lq=16, Lk=16, Hq=2, Hkv=1, D=128, qv=16, kv=16, causal=1,
             scale=0.1, mods=None, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize(
    "over,msg",
    [
        (dict(dtype=7), "dtype"),
        (dict(q=None), "non-null"),
        (dict(D=96), "head_dim"),
        (dict(Hq=3, Hkv=2), "multiple of kv_heads"),
        (dict(scale=0.0), "sm_scale"),
        (dict(bias=1, bb=3), "bias"),
        (dict(B=-1), "negative"),
    ],
)
def test_flash_rejects_invalid_arguments(lib, over, msg):
    rc = lib.pjx_flash_fwd(*_flash_args(**over))
    assert rc == 1
    assert msg in lib.pjx_last_error().decode()


@pytest.mark.parametrize(
    "fields,msg",
    [
        (dict(softcap=-1.0), "softcap"),
        (dict(softcap=5.0, head_scales=1), "exclude"),
        (dict(segment_q=1), "segment_q and segment_k"),
        (dict(segment_q=1, segment_k=1, row_kv_lengths=1), "row_kv_lengths excludes"),
        (dict(window_left=0x3FFFFFFF), "out of range"),
    ],
)
def test_flash_rejects_invalid_score_mods(lib, fields, msg):
    m = native.ScoreMods(**{"window_left": -1, "window_right": -1, **fields})
    for fn, args in (("pjx_flash_fwd", _flash_args(mods=ctypes.pointer(m))),
                     ("pjx_flash_bwd", _bwd_args(mods=ctypes.pointer(m)))):
        assert getattr(lib, fn)(*args) == 1, fn
        assert msg in lib.pjx_last_error().decode(), fn


def _bwd_args(**over):
    a = dict(dtype=native.PJX_DTYPE_BF16, q=1, k=1, v=1, o=1, do=1, lse=1, dq=1, dk=1, dv=1,
             dbias=None, ws=1, ws_bytes=1 << 20, kvl=None, bias=None, bb=1, bh=1, B=1, Lq=16, Lk=16, Hq=2,
             Hkv=1, D=128, qv=16, kv=16, causal=1, scale=0.1, mods=None, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize(
    "over,msg,code",
    [
        (dict(dtype=7), "dtype", 1),
        (dict(do=None), "non-null", 1),
        (dict(dbias=1), "dbias needs the bias", 1),
        (dict(D=96), "head_dim", 1),
        (dict(Hq=3, Hkv=2), "multiple of kv_heads", 1),
        (dict(ws=None), "workspace", 3),
        (dict(ws_bytes=16), "workspace", 3),
    ],
)
def test_flash_bwd_rejects_invalid_arguments(lib, over, msg, code):
    assert lib.pjx_flash_bwd(*_bwd_args(**over)) == code
    assert msg in lib.pjx_last_error().decode()


def test_flash_bwd_workspace_size(lib):
    assert lib.pjx_flash_bwd_workspace_size(2, 3, 5) == 8 * 2 * 3 * 5
    assert lib.pjx_flash_bwd_workspace_size(0, 3, 5) == 0


def test_flash_bwd_ds_workspace_size(lib):
    """The dS route exists for 16-bit inputs at head dim 256 only; its
    workspace is the plain one rounded up to 256 bytes plus 1 KiB per block of
    32 queries x 16 keys per head, both lengths rounded up to 64."""
    bf16, f16, f32 = native.PJX_DTYPE_BF16, native.PJX_DTYPE_F16, native.PJX_DTYPE_F32
    B, H, Lq, Lk = 2, 3, 300, 70
    base = lib.pjx_flash_bwd_workspace_size(B, H, Lq)
    lead = (base + 255) // 256 * 256
    nq32, nk16 = 2 * ((Lq + 63) // 64), 4 * ((Lk + 63) // 64)
    for dt in (bf16, f16):
        assert lib.pjx_flash_bwd_ds_workspace_size(dt, B, H, Lq, Lk, 256) == lead + B * H * nq32 * nk16 * 1024
    for dt, d in ((f32, 256), (bf16, 128), (bf16, 64), (f16, 128)):
        assert lib.pjx_flash_bwd_ds_workspace_size(dt, B, H, Lq, Lk, d) == 0
    assert lib.pjx_flash_bwd_ds_workspace_size(bf16, 0, H, Lq, Lk, 256) == 0
    assert lib.pjx_flash_bwd_ds_workspace_size(bf16, B, H, Lq, 0, 256) == 0


def test_flash_empty_batch_is_a_no_op(lib):
    assert lib.pjx_flash_fwd(*_flash_args(B=0)) == 0


def test_decode_rejects_invalid_arguments(lib):
    P = ctypes.c_void_p
    ok = [native.PJX_DTYPE_BF16, P(1), P(1), P(1), None, P(1), None, P(1), 1 << 30,
          1, 1, 64, 32, 8, 128, 128, 0.1, 0, None]
    bad_dim = list(ok)
    bad_dim[14] = 96  # head dims 64, 128, 256
    assert lib.pjx_splitkv_decode(*bad_dim) == 1
    assert "head_dim and v_dim" in lib.pjx_last_error().decode()
    bad_vdim = list(ok)
    bad_vdim[15] = 512
    assert lib.pjx_splitkv_decode(*bad_vdim) == 1
    assert "head_dim and v_dim" in lib.pjx_last_error().decode()
    bad_chunk = list(ok)
    bad_chunk[17] = 100
    assert lib.pjx_splitkv_decode(*bad_chunk) == 1
    assert "chunk" in lib.pjx_last_error().decode()
    bad_dtype = list(ok)
    bad_dtype[0] = 7
    assert lib.pjx_splitkv_decode(*bad_dtype) == 1
    assert "dtype" in lib.pjx_last_error().decode()
    bad_heads = list(ok)
    bad_heads[12] = 30  # Hq not a multiple of Hkv
    assert lib.pjx_splitkv_decode(*bad_heads) == 1
    mla = [native.PJX_DTYPE_BF16, P(1), P(1), None, P(1), None, P(1), 1 << 30,
           1, 1, 16, 64, 300, 512, 0.1, 0, None]
    assert lib.pjx_mla_decode(*mla) == 1
    assert "rank" in lib.pjx_last_error().decode() or "supported" in lib.pjx_last_error().decode()


def test_static_decode_checks_arguments_before_size(lib):
    """pjx_splitkv_decode_static runs every argument check of
    pjx_splitkv_decode before sizing its partials: a bad head dim or chunk is
    PJX_ERR_INVALID whatever the sizes, and B = 0 with a bad dtype is refused."""
    big = [1, None, None, None, None, None, None, 256, 1, 1 << 20, 16, 16]
    for dt, d, dv, chunk, msg in ((native.PJX_DTYPE_BF16, 96, 128, 0, "head_dim"),
                                  (native.PJX_DTYPE_BF16, 128, 128, 100, "chunk"),
                                  (7, 128, 128, 0, "dtype")):
        args = list(big)
        args[0] = dt
        assert lib.pjx_splitkv_decode_static(*args, d, dv, 0.1, chunk, None) == 1
        assert msg in lib.pjx_last_error().decode()
    zero_batch = [7, None, None, None, None, None, None, 0, 1, 100, 8, 8, 128, 128, 0.1, 0, None]
    assert lib.pjx_splitkv_decode_static(*zero_batch) == 1


def test_workspace_size_formula(lib):
    # partial outputs + (max, sum) per (batch, group, chunk, row), fp32
    n = lib.pjx_decode_workspace_size(2, 8, 4, 1000, 128, 256)
    chunks = -(-1000 // 256)
    assert n == 2 * 8 * chunks * 4 * (128 + 2) * 4


def test_launch_log_empty_after_refused_call(lib):
    """A call refused before any launch leaves an empty launch log (the log
    of a call lists the kernel instances it launched, in order)."""
    rc = lib.pjx_flash_fwd(*_flash_args(D=96))
    assert rc != native.PJX_OK
    assert lib.pjx_last_launches() == b""
    assert native.last_launches() == []
