"""The two C-ABI libraries load and export every function their headers
declare, and the GPU library's host-side validation (no GPU work) rejects bad
parameters with the documented codes. CPU only."""
import ctypes as ct
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "astc-kv_amd" / "astc_kv"
LIBS = {"astc_kv.h": PKG / "libakv_astc.so", "astc_kv_hip.h": PKG / "libastckv_hip.so"}


def declared_functions(header: Path):
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(akv_\w+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(LIBS))
def test_library_exports_every_declared_function(header):
    lib_path = LIBS[header]
    assert lib_path.exists(), f"{lib_path} missing: run astc-kv_amd/build.py"
    names = declared_functions(ROOT / "include" / header)
    assert len(names) >= 5
    lib = ct.CDLL(str(lib_path))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"{lib_path.name} lacks {missing}"


class Params(ct.Structure):
    _fields_ = [(name, ct.c_uint32) for name in (
        "batch", "tokens", "query_heads", "kv_heads", "dim", "page_tokens", "tile_tokens", "splits",
        "layout", "block_x", "block_y", "atlas_rows", "atlas_cols")]


@pytest.fixture(scope="module")
def hip():
    lib = ct.CDLL(str(LIBS["astc_kv_hip.h"]))
    lib.akv_hip_task_tokens.argtypes = [ct.POINTER(Params), ct.c_int]
    lib.akv_hip_task_tokens.restype = ct.c_int
    lib.akv_hip_error_string.argtypes = [ct.c_int]
    lib.akv_hip_error_string.restype = ct.c_char_p
    return lib


def c3(**kw):
    """T8192 batch 16, 9q/3kv, D64, RGBA 6x5 atlas padded to pages of 120 tokens."""
    p = dict(batch=16, tokens=8192, query_heads=9, kv_heads=3, dim=64, page_tokens=120, tile_tokens=240,
             splits=35, layout=1, block_x=6, block_y=5, atlas_rows=1656, atlas_cols=3)
    p.update(kw)
    return Params(**p)


def test_chunk_tokens_follow_the_footprint(hip):
    # Launches of more workgroups than CUs (16 splits x 3 kv heads x batch 16
    # = 768): at head dim 64 a chunk holds at most 160 blocks.
    big = dict(tile_tokens=512, splits=16)
    # 6x5 RGBA D64: 3 block columns -> 53 block rows; a chunk starts on a
    # 16-token boundary, at most 4 tokens into its first row, so 261 tokens
    # fit; 256 = 16 tiles, the same number for every wave.
    assert hip.akv_hip_task_tokens(ct.byref(c3(**big)), 1) == 256
    # A split shorter than a chunk is one chunk.
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=48, splits=171)), 1) == 48
    # 4x4 RGBA D64: 4 block columns -> 40 block rows = 160 tokens.
    p = c3(block_x=4, block_y=4, atlas_cols=4, atlas_rows=2048, **big)
    assert hip.akv_hip_task_tokens(ct.byref(p), 1) == 160
    # Scalar 6x6 D64: 11 block columns -> 14 rows = 84 tokens, at most 4 in
    # at the start -> 80.
    p = c3(layout=0, block_x=6, block_y=6, atlas_cols=11, atlas_rows=1366, **big)
    assert hip.akv_hip_task_tokens(ct.byref(p), 1) == 80
    # At most one workgroup per CU (1 split x 48): the wide kernel's 256-block
    # chunks. 6x5: 85 rows, capped at 320 tokens -> 256; 4x4: 64 rows = 256;
    # scalar 6x6: 23 rows = 138 tokens, 4 in at the start -> 128.
    one = dict(tile_tokens=8192, splits=1)
    assert hip.akv_hip_task_tokens(ct.byref(c3(**one)), 1) == 256
    p = c3(block_x=4, block_y=4, atlas_cols=4, atlas_rows=2048, **one)
    assert hip.akv_hip_task_tokens(ct.byref(p), 1) == 256
    p = c3(layout=0, block_x=6, block_y=6, atlas_cols=11, atlas_rows=1366, **one)
    assert hip.akv_hip_task_tokens(ct.byref(p), 1) == 128
    # D128 RGBA 4x4: 8 block columns, at most 256 blocks -> 32 rows = 128 tokens.
    p = c3(dim=128, block_x=4, block_y=4, atlas_cols=8, atlas_rows=2048, tile_tokens=8192, splits=1)
    assert hip.akv_hip_task_tokens(ct.byref(p), 1) == 128
    # Any tile is legal (probe_gqa_v10.mm:466). Chunks then start at any token,
    # at most by - gcd(16, tile, by) tokens into their first block row.
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=238, splits=35)), 1) == 238
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=1, splits=8192)), 1) == 1
    s66 = dict(layout=0, block_x=6, block_y=6, atlas_cols=11, atlas_rows=1366)
    # scalar 6x6: tile 200 -> starts are even, at most 4 in -> 84 - 4 = 80;
    # tile 201 -> at most 5 in -> 79 -> whole tiles: 64.
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=200, splits=41, **s66)), 1) == 80
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=201, splits=41, **s66)), 1) == 64
    # FP16 control: whole 320-token chunks (128 for D128).
    assert hip.akv_hip_task_tokens(ct.byref(c3(tile_tokens=8192, splits=1)), 0) == 320
    assert hip.akv_hip_task_tokens(ct.byref(c3(dim=128, tile_tokens=8192, splits=1)), 0) == 128


@pytest.mark.parametrize("kw,code", [
    (dict(dim=96), -2),                               # head dim not 64/128
    (dict(query_heads=10), -2),                       # Hq not a multiple of Hkv
    (dict(query_heads=15, kv_heads=3), -2),           # G = 5 unsupported
    (dict(batch=0), -2),
    (dict(atlas_cols=4), -2),                         # atlas width inconsistent with dim/layout/footprint
    (dict(atlas_rows=1000), -2),                      # atlas shorter than the sequence
    (dict(layout=7), -2),
    (dict(block_x=3), -3),                            # footprint below 4
    (dict(block_x=10, block_y=8, atlas_cols=2), -3),  # more than 64 texels
    (dict(splits=34), -4),                            # splits != ceil(T / tile)
    (dict(tile_tokens=0), -4),
])
def test_rejected_parameters(hip, kw, code):
    assert hip.akv_hip_task_tokens(ct.byref(c3(**kw)), 1) == code
    assert hip.akv_hip_error_string(code).decode() != "unknown error"


@pytest.mark.parametrize("bad", ["q", "k", "v"])
def test_misaligned_pointers_rejected_before_any_launch(hip, bad):
    # Fake device addresses: the argument checks return before anything is
    # dereferenced or launched, so this runs without a GPU.
    fn = hip.akv_hip_decode_attention
    fn.argtypes = [ct.POINTER(Params)] + [ct.c_void_p] * 9
    fn.restype = ct.c_int
    ptr = {"q": 0x10000, "k": 0x20000, "v": 0x30000}
    ptr[bad] += 4
    args = [ptr["q"], ptr["k"], ptr["v"], 0x40000, 0x50000, 0x60000, 0x70000, 0x80000, None]
    assert fn(ct.byref(c3(tile_tokens=512, splits=16)), *args) == -5
    assert b"16-byte" in hip.akv_hip_error_string(-5)


class PagedParams(ct.Structure):
    _fields_ = [(name, ct.c_uint32) for name in (
        "batch", "max_tokens", "query_heads", "kv_heads", "dim", "page_tokens", "max_pages", "num_pages",
        "tile_tokens", "splits", "layout", "block_x", "block_y", "atlas_cols", "k_format")]


def test_append_and_commit_validation(hip):
    # Host-side checks only (no launch): fake device addresses.
    ap, cm = hip.akv_hip_paged_append, hip.akv_hip_paged_commit_pages
    ap.argtypes = [ct.POINTER(PagedParams)] + [ct.c_void_p] * 8
    cm.argtypes = [ct.POINTER(PagedParams), ct.c_uint32] + [ct.c_void_p] * 8
    ap.restype = cm.restype = ct.c_int
    p = PagedParams(batch=4, max_tokens=1000, query_heads=32, kv_heads=8, dim=128, page_tokens=96, max_pages=12,
                    num_pages=48, tile_tokens=0, splits=0, layout=0, block_x=6, block_y=6, atlas_cols=22,
                    k_format=1)
    a = [0x10000 * (i + 1) for i in range(8)]
    assert ap(None, *a) == -1
    # arguments: k_new, v_new, k_pages, k_meta, block_table, seq_lens, v_tail, stream
    assert ap(ct.byref(p), *(a[:6] + [None] + a[7:])) == -1         # the FP16 tail is required
    assert ap(ct.byref(p), *(a[:3] + [None] + a[4:])) == -1         # 4-bit K needs k_meta
    bad = PagedParams.from_buffer_copy(p)
    bad.atlas_cols = 21
    assert ap(ct.byref(bad), *a) == -2
    bad = PagedParams.from_buffer_copy(p)
    bad.page_tokens = 90                                            # not a multiple of 16
    assert cm(ct.byref(bad), 1, *a) == -2
    assert cm(ct.byref(p), 0, *a) == 0                              # nothing to copy
    # arguments: page_ids, blocks, scale, offset, v_blocks, v_scale, v_offset, stream
    assert cm(ct.byref(p), 1, *(a[:2] + [a[2] + 8] + a[3:])) == -5   # staging scale not 16-byte aligned


def test_null_params_and_error_strings(hip):
    assert hip.akv_hip_task_tokens(None, 1) == -1
    assert hip.akv_hip_error_string(0) == b"success"
    assert b"NULL" in hip.akv_hip_error_string(-1)
    assert hip.akv_hip_error_string(-99) == b"unknown error"


def test_bridge_error_strings_and_context():
    lib = ct.CDLL(str(LIBS["astc_kv.h"]))
    lib.akv_create.argtypes = [ct.c_uint, ct.c_uint, ct.c_float, ct.c_int, ct.POINTER(ct.c_int)]
    lib.akv_create.restype = ct.c_void_p
    lib.akv_destroy.argtypes = [ct.c_void_p]
    lib.akv_error.argtypes = [ct.c_int]
    lib.akv_error.restype = ct.c_char_p
    err = ct.c_int(-1)
    ctx = lib.akv_create(6, 5, 50.0, 0, ct.byref(err))
    assert ctx and err.value == 0
    lib.akv_destroy(ctx)
    err = ct.c_int(0)
    assert not lib.akv_create(3, 3, 50.0, 0, ct.byref(err)) and err.value != 0
    assert lib.akv_error(err.value)
    err = ct.c_int(0)
    assert not lib.akv_create(6, 6, 50.0, 1, ct.byref(err)) and err.value != 0   # HDR profile: LDR-only codec
