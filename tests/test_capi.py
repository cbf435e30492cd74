"""The C-ABI library without a GPU: it loads, exports every function that
``include/mstar_amd.h`` declares with the argument count the ctypes binding
uses, sizes workspaces on the host, and rejects invalid arguments before any
HIP call (every call below returns from argument validation, so none touches
a device).
"""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from mstar_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "mstar_amd.h"

MI_ERR_INVALID = -1
MI_ERR_UNSUPPORTED = -2


def _declared():
    """name -> number of parameters, from the prototypes in the header."""
    text = re.sub(r"/\*.*?\*/|//[^\n]*", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"\b(mi_[a-z0-9_]+)\s*\(([^;{)]*)\)\s*;", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_header_declares_the_bound_functions():
    decl = _declared()
    assert set(decl) == set(_lib.SIGNATURES)
    for name, nargs in decl.items():
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def test_library_exports_every_declared_symbol(L):
    res = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True)
    exported = {ln.split()[-1] for ln in res.stdout.splitlines() if ln.strip()}
    for name in _declared():
        assert name in exported, name
        assert getattr(L, name) is not None


def test_abi_version_and_status_strings(L):
    assert L.mi_abi_version() == _lib.ABI_VERSION
    for code, text in [(0, b"ok"), (-1, b"invalid argument")]:
        assert L.mi_status_string(code) == text
    for code in (-2, -3, -4, 12345):
        assert L.mi_status_string(code)


def test_workspace_sizes_are_host_arithmetic(L):
    d = L.mi_decode_workspace_bytes(256, 32, 4, 128)
    assert d > 0 and d % 256 == 0
    # per item the workspace holds at least the fp32 partial output of every kv-head
    assert d >= 256 * 4 * 16 * 128 * 4
    assert L.mi_decode_workspace_bytes(512, 32, 4, 128) > d
    p = L.mi_prefill_workspace_bytes(8, 4096, 32, 4, 128)
    assert p > 0 and p % 256 == 0
    assert L.mi_prefill_workspace_bytes(8, 8192, 32, 4, 128) > p
    assert L.mi_decode_workspace_bytes(-1, 32, 4, 128) < 0
    assert L.mi_prefill_workspace_bytes(8, 4096, 32, 5, 128) < 0  # 32 % 5 != 0


def test_prefill_short_rows(L):
    """Short-query threshold: 16 rows, 8 on plans that read kv-head pairs
    (batch >= 128, head_dim 128, group <= 8, even kv-head count)."""
    assert L.mi_prefill_short_rows(8, 28, 4, 128) == 16      # batch below 128
    assert L.mi_prefill_short_rows(128, 28, 4, 128) == 8     # c4's shape: paired
    assert L.mi_prefill_short_rows(200, 32, 4, 256) == 16    # head_dim 256
    assert L.mi_prefill_short_rows(200, 36, 4, 128) == 16    # group 9: a pair's rows exceed 16
    assert L.mi_prefill_short_rows(200, 24, 3, 128) == 16    # odd kv-head count
    assert L.mi_prefill_short_rows(200, 30, 4, 128) < 0      # heads not a multiple


def test_invalid_arguments_are_rejected_before_launch(L):
    nul = None
    # negative batch, null outputs
    assert L.mi_pack(nul, nul, nul, nul, -1, nul, 0, nul, nul, 16, nul, nul, nul, nul, nul, 1, nul) == MI_ERR_INVALID
    assert L.mi_block_table_update(nul, 0, nul, nul, nul, 4, nul) == MI_ERR_INVALID
    # null workspace
    assert L.mi_decode_plan(nul, nul, nul, nul, 4, 16, 32, 4, 128, nul, nul, 0, nul) == MI_ERR_INVALID


def test_unsupported_shapes_are_reported(L):
    buf = (ctypes.c_int32 * 8)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    # GQA group 32 > 16 rows per wavefront, page size not a multiple of 16, head_dim 96
    assert L.mi_decode_plan(p, p, p, p, 1, 16, 32, 1, 128, None, p, 1 << 30, None) == MI_ERR_UNSUPPORTED
    assert L.mi_decode_plan(p, p, p, p, 1, 8, 32, 4, 128, None, p, 1 << 30, None) == MI_ERR_UNSUPPORTED
    assert L.mi_decode_plan(p, p, p, p, 1, 16, 32, 4, 96, None, p, 1 << 30, None) == MI_ERR_UNSUPPORTED



def test_pack_plan_arguments_are_checked(L):
    """mi_pack_plan: the pack's checks, then the decode plan's (heads, head_dim, workspace)."""
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    MI_ERR_WORKSPACE = -3

    def call(batch=4, grid=1, hq=32, hkv=4, d=128, ws=p, ws_bytes=1 << 30, ps=16):
        return L.mi_pack_plan(p, p, p, p, batch, p, 8, None, None, ps, p, p, p, p, None, grid, hq, hkv, d, ws,
                              ws_bytes, None)

    assert call(batch=-1) == MI_ERR_INVALID           # pack: negative batch
    assert call(grid=0) == MI_ERR_INVALID             # pack: no workgroups
    assert call(ws=None) == MI_ERR_INVALID            # plan: no workspace
    assert call(hq=30, hkv=4) == MI_ERR_INVALID       # plan: heads not a multiple
    assert call(hq=64, hkv=2) == MI_ERR_UNSUPPORTED   # plan: GQA group 32 > 16
    assert call(d=96) == MI_ERR_UNSUPPORTED           # plan: head_dim
    assert call(ps=8) == MI_ERR_UNSUPPORTED           # plan: page size not a multiple of 16
    assert call(ws_bytes=1024) == MI_ERR_WORKSPACE    # plan: workspace too small


def test_rope_arguments_are_checked(L):
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    # rotary_dim not a multiple of 8, rotary_dim > head_dim, fp32 tensors, zero rope_scale
    assert L.mi_rope_apply(p, 128, 128, 1, p, 128, 128, 1, 0, 128, 12, p, 4, 1, 0, 1.0, 1e4, 0, 1.0, 4.0, 8192.0,
                           None) == MI_ERR_UNSUPPORTED
    assert L.mi_rope_apply(p, 128, 128, 1, p, 128, 128, 1, 0, 64, 128, p, 4, 1, 0, 1.0, 1e4, 0, 1.0, 4.0, 8192.0,
                           None) == MI_ERR_UNSUPPORTED
    assert L.mi_rope_apply(p, 128, 128, 1, p, 128, 128, 1, 2, 128, 128, p, 4, 1, 0, 1.0, 1e4, 0, 1.0, 4.0, 8192.0,
                           None) == MI_ERR_UNSUPPORTED
    assert L.mi_rope_apply(p, 128, 128, 1, p, 128, 128, 1, 0, 128, 128, p, 4, 1, 0, 0.0, 1e4, 0, 1.0, 4.0, 8192.0,
                           None) == MI_ERR_INVALID
    # llama31 needs high > low > 0
    assert L.mi_rope_apply(p, 128, 128, 1, p, 128, 128, 1, 0, 128, 128, p, 4, 1, 0, 8.0, 5e5, 1, 4.0, 1.0, 8192.0,
                           None) == MI_ERR_INVALID
    assert L.mi_rope_positions(None, None, 0, None, 5, None) == MI_ERR_INVALID
    assert L.mi_rope_positions(None, None, 0, None, 0, None) == 0


def test_rope_append_arguments_are_checked(L):
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)

    def kv(**kw):
        d = _lib.MiPagedKV()
        d.data, d.dtype, d.page_size, d.num_kv_heads, d.head_dim = 4096, 0, 16, 2, 128
        d.max_pages, d.page_stride, d.kv_stride, d.token_stride, d.head_stride = 8, 8192, 4096, 256, 128
        for k, v in kw.items():
            setattr(d, k, v)
        return ctypes.byref(d)

    def call(desc, rd=128, dtype=0, k_stride=256, scale=1.0, llama=(0, 1.0, 4.0), ntok=3, nappend=3, pos=p):
        return L.mi_rope_append(p, 512, 128, 4, p, k_stride, 128, p, 256, 128, dtype, 1, desc, p, p, 1, nappend,
                                None, rd, pos, 5, ntok, 0, scale, 1e4, llama[0], llama[1], llama[2], 8192.0, None)

    assert call(kv(), ntok=0) == 0                                      # nothing to do
    assert call(kv(), nappend=-1) == MI_ERR_INVALID
    assert call(None) == MI_ERR_INVALID
    assert call(kv(), pos=None) == MI_ERR_INVALID
    assert call(kv(), rd=12) == MI_ERR_UNSUPPORTED                      # rotary_dim % 8
    assert call(kv(), rd=256) == MI_ERR_UNSUPPORTED                     # rotary_dim > head_dim
    assert call(kv(), dtype=2) == MI_ERR_UNSUPPORTED                    # fp32 q/k/v
    assert call(kv(dtype=3)) == MI_ERR_INVALID                          # fp8 cache without scales
    assert call(kv(), scale=0.0) == MI_ERR_INVALID
    assert call(kv(), llama=(1, 4.0, 1.0)) == MI_ERR_INVALID            # high <= low
    assert call(kv(), k_stride=260) == MI_ERR_INVALID                   # k rows not 8-element aligned
    assert call(kv(token_stride=260)) == MI_ERR_INVALID                 # cache rows not 8-element aligned
    assert call(kv(data=4100)) == MI_ERR_INVALID                        # cache base not 16-byte aligned


def test_transfer_arguments_are_checked(L):
    """KV transfer: malformed pool descriptors and ranges fail before any HIP call."""
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)

    def pool(**kw):
        d = _lib.MiKvPool()
        d.data, d.layer_stride, d.page_stride, d.kv_stride, d.token_stride = 4096, 1 << 20, 1 << 14, 1 << 13, 512
        d.num_pages, d.num_layers, d.page_size = 16, 2, 16
        for k, v in kw.items():
            setattr(d, k, v)
        return ctypes.byref(d)

    bad = [pool(data=None), pool(token_stride=0), pool(page_stride=24), pool(data=4100), pool(kv_stride=256),
           pool(num_layers=0)]
    for b in bad:
        assert L.mi_kv_copy_tokens(b, b, p, p, None, None, 1, 0, 1, None) == MI_ERR_INVALID
        assert L.mi_kv_wire_pack(b, p, None, None, None, 1, 0, 1, p, 64, None) == MI_ERR_INVALID
        assert L.mi_kv_wire_unpack(p, 64, b, p, None, None, None, 1, 0, 1, None) == MI_ERR_INVALID
    good = pool()
    assert L.mi_kv_copy_tokens(None, good, p, p, None, None, 1, 0, 1, None) == MI_ERR_INVALID
    # layer range past the pool, negative record count, one-sided token range
    assert L.mi_kv_copy_tokens(good, good, p, p, None, None, 1, 0, 3, None) == MI_ERR_INVALID
    assert L.mi_kv_copy_tokens(good, good, p, p, None, None, -1, 0, 1, None) == MI_ERR_INVALID
    assert L.mi_kv_copy_tokens(good, good, p, p, p, None, 1, 0, 1, None) == MI_ERR_INVALID
    assert L.mi_kv_wire_pack(good, p, p, None, None, 1, 0, 1, p, 64, None) == MI_ERR_INVALID
    # the HBM read probe: null buffers, sizes that are not whole 16-byte pieces, misalignment, no grid
    assert L.mi_hbm_read(None, 16, p, 1, None) == MI_ERR_INVALID
    assert L.mi_hbm_read(p, 16, None, 1, None) == MI_ERR_INVALID
    assert L.mi_hbm_read(p, 20, p, 1, None) == MI_ERR_INVALID
    assert L.mi_hbm_read(4100, 16, p, 1, None) == MI_ERR_INVALID
    assert L.mi_hbm_read(p, 0, p, 1, None) == MI_ERR_INVALID
    assert L.mi_hbm_read(p, 16, p, 0, None) == MI_ERR_INVALID


def test_noalloc_decode_rejects_oversized_batch_on_the_host(L):
    """mi_decode_noalloc checks the batch against its fixed device buffer before any HIP call."""
    d = _lib.MiPagedKV()
    d.data, d.dtype, d.page_size, d.num_kv_heads, d.head_dim = 4096, 0, 16, 4, 128
    buf = (ctypes.c_int32 * 8)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    MI_ERR_WORKSPACE = -3
    # about 33 KB of partials per split-KV item at 4 kv heads x head_dim 128: 4000 + 1 items exceed 64 MiB
    assert L.mi_decode_noalloc(p, 0, 4096, 128, ctypes.byref(d), None, p, p, p, 4000, 32, 0, 0.1, p, 4096, 128,
                               None, None) == MI_ERR_WORKSPACE
    assert L.mi_decode_noalloc(p, 0, 4096, 128, None, None, p, p, p, 4, 32, 0, 0.1, p, 4096, 128, None,
                               None) == MI_ERR_INVALID
    assert L.mi_decode_noalloc(p, 0, 4096, 128, ctypes.byref(d), None, p, p, p, 0, 32, 0, 0.1, p, 4096, 128, None,
                               None) == 0


def test_attention_entry_points_reject_unaligned_rows_on_the_host(L):
    """q / out / KV rows that are not 16-byte pieces are rejected before any HIP call."""
    d = _lib.MiPagedKV()
    d.data, d.dtype, d.page_size, d.num_kv_heads, d.head_dim = 4096, 0, 16, 4, 128
    d.page_stride, d.kv_stride, d.token_stride, d.head_stride = 2 * 16 * 4 * 128, 16 * 4 * 128, 4 * 128, 128
    d.max_pages = 64
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    ws = ctypes.c_void_p(base)
    ok_q, bad_q = ctypes.c_void_p(base), ctypes.c_void_p(base + 2)
    for name in ("mi_decode_run", "mi_decode_attend", "mi_decode_merge"):
        fn = getattr(L, name)
        # q base off by one element, q token stride of 4 elements, out head stride of 12 elements
        assert fn(bad_q, 0, 4096, 128, ctypes.byref(d), None, p, p, p, 4, 32, 0, 0.1, ws, 1 << 20, ok_q, 4096,
                  128, None) == MI_ERR_INVALID
        assert fn(ok_q, 0, 4, 128, ctypes.byref(d), None, p, p, p, 4, 32, 0, 0.1, ws, 1 << 20, ok_q, 4096, 128,
                  None) == MI_ERR_INVALID
        assert fn(ok_q, 0, 4096, 128, ctypes.byref(d), None, p, p, p, 4, 32, 0, 0.1, ws, 1 << 20, ok_q, 4096, 12,
                  None) == MI_ERR_INVALID
    bad = _lib.MiPagedKV.from_buffer_copy(d)
    bad.head_stride = 132  # KV rows of 264 bytes
    assert L.mi_decode_run(ok_q, 0, 4096, 128, ctypes.byref(bad), None, p, p, p, 4, 32, 0, 0.1, ws, 1 << 20, ok_q,
                           4096, 128, None) == MI_ERR_INVALID
    assert L.mi_prefill_run(bad_q, 0, 4096, 128, ctypes.byref(d), p, p, p, p, 4, 64, 32, 1, 0.1, ws, 1 << 20,
                            ok_q, 4096, 128, None) == MI_ERR_INVALID
    assert L.mi_prefill_run(ok_q, 0, 4096, 128, ctypes.byref(bad), p, p, p, p, 4, 64, 32, 1, 0.1, ws, 1 << 20,
                            ok_q, 4096, 128, None) == MI_ERR_INVALID
    # K and V halves 2^31 bytes apart: beyond the prefill loader's 32-bit in-page offsets
    far = _lib.MiPagedKV.from_buffer_copy(d)
    far.kv_stride = 1 << 30
    far.page_stride = 2 * far.kv_stride
    assert L.mi_prefill_run(ok_q, 0, 4096, 128, ctypes.byref(far), p, p, p, p, 4, 64, 32, 1, 0.1, ws, 1 << 20,
                            ok_q, 4096, 128, None) == MI_ERR_UNSUPPORTED


def test_pack_plan_host_arguments_are_checked(L):
    """mi_pack_plan_host: the metadata size against the argument buffer, then mi_pack_plan's checks."""
    meta = (ctypes.c_int32 * 1024)()
    m = ctypes.cast(meta, ctypes.c_void_p)
    buf = (ctypes.c_int32 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)

    def call(meta_len=20, batch=4, grid=1, ws=p, meta_ptr=m):
        return L.mi_pack_plan_host(meta_ptr, meta_len, batch, p, 8, 16, p, p, p, p, None, grid, 32, 4, 128, ws,
                                   1 << 30, None)

    assert call(meta_len=4097) == MI_ERR_INVALID       # more than MI_PACK_HOST_META_MAX values
    meta[12] = 3                                       # request 0 holds 3 pages, none in the table:
    assert call(meta_len=20) == MI_ERR_INVALID         # 3 new pages expected, none given
    meta[12] = 0
    assert call(meta_len=19) == MI_ERR_INVALID         # fewer than 5 values per request
    assert call(meta_ptr=None) == MI_ERR_INVALID       # no metadata
    assert call(grid=0) == MI_ERR_INVALID              # pack: no workgroups
    assert call(grid=0, ws=None) == MI_ERR_INVALID     # pack only: same checks

    # beyond MI_PACK_HOST_ARGS values: only a step that fits the compact form is launched
    big = (ctypes.c_int32 * 4096)()
    bm = ctypes.cast(big, ctypes.c_void_p)
    assert call(meta_len=5 * 300, batch=300, meta_ptr=bm) == MI_ERR_UNSUPPORTED  # 3 * 300 > 896 values
    big[0] = 70000                                                             # a slot above 2^16
    assert call(meta_len=5 * 200, batch=200, meta_ptr=bm) == MI_ERR_UNSUPPORTED
    big[0] = 0
    big[3 * 200] = 2                                                           # 2 pages, 2 new ones given
    assert call(meta_len=5 * 200 + 1, batch=200, meta_ptr=bm) == MI_ERR_INVALID  # counts disagree
