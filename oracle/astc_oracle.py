"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py's
CPU-baseline leg). Never imported by the product package.

ctypes binding of oracle/astc_oracle.c, the CPU restatement of astcenc's LDR
block decode (reference call sites: astc_kv/bridge.cpp:27-35, astc_kv/codec.py:56).
"""
from __future__ import annotations

import ctypes as ct
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None


def build() -> Path:
    """Compile the oracle's C restatement in place (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _HERE / "liboracle_astc.so"


def lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "liboracle_astc.so"
        if not path.exists() or path.stat().st_mtime < (_HERE / "astc_oracle.c").stat().st_mtime:
            build()
        L = ct.CDLL(str(path))
        L.oracle_decode_blocks_fp16.argtypes = [ct.c_void_p, ct.c_long, ct.c_int, ct.c_int, ct.c_void_p, ct.c_void_p]
        L.oracle_decode_block_unorm16.argtypes = [ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p]
        L.oracle_decode_block_unorm16.restype = ct.c_int
        L.oracle_decode_image.argtypes = [ct.c_void_p, ct.c_long, ct.c_int, ct.c_int, ct.c_int, ct.c_int, ct.c_void_p]
        L.oracle_decode_image.restype = ct.c_int
        L.oracle_unorm16_to_fp16.argtypes = [ct.c_uint]
        L.oracle_unorm16_to_fp16.restype = ct.c_uint16
        L.oracle_select_partition.argtypes = [ct.c_int] * 6
        L.oracle_select_partition.restype = ct.c_int
        L.oracle_unquant_color.argtypes = [ct.c_int, ct.c_int]
        L.oracle_unquant_color.restype = ct.c_int
        L.oracle_unquant_weight.argtypes = [ct.c_int, ct.c_int]
        L.oracle_unquant_weight.restype = ct.c_int
        L.oracle_ise_bits.argtypes = [ct.c_int, ct.c_int]
        L.oracle_ise_bits.restype = ct.c_int
        L.oracle_decode_trits.argtypes = [ct.c_uint, ct.c_void_p]
        L.oracle_decode_quints.argtypes = [ct.c_uint, ct.c_void_p]
        _LIB = L
    return _LIB


def decode_blocks_fp16(blocks: np.ndarray, bx: int, by: int):
    """blocks: uint8 [n,16] -> (fp16 [n,by,bx,4], kinds int32 [n])."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 16)
    n = len(blocks)
    out = np.empty((n, by, bx, 4), np.float16)
    kinds = np.empty(n, np.int32)
    lib().oracle_decode_blocks_fp16(blocks.ctypes.data, n, bx, by, out.ctypes.data, kinds.ctypes.data)
    return out, kinds


def decode_block_unorm16(block: bytes, bx: int, by: int):
    out = np.empty((by, bx, 4), np.uint16)
    buf = np.frombuffer(bytes(block), np.uint8).copy()
    kind = lib().oracle_decode_block_unorm16(buf.ctypes.data, bx, by, out.ctypes.data)
    return out, kind


def decode_image(payload: bytes, bx: int, by: int, width: int, height: int) -> np.ndarray:
    """Row-major block payload -> float32 RGBA image [height, width, 4]."""
    buf = np.frombuffer(bytes(payload), np.uint8).copy()
    img = np.empty((height, width, 4), np.float32)
    if lib().oracle_decode_image(buf.ctypes.data, len(buf), bx, by, width, height, img.ctypes.data):
        raise ValueError("payload too short for image")
    return img


def unorm16_to_fp16(c: int) -> int:
    return int(lib().oracle_unorm16_to_fp16(c))


def select_partition(seed: int, x: int, y: int, z: int, count: int, small: bool) -> int:
    return int(lib().oracle_select_partition(seed, x, y, z, count, int(small)))


def unquant_color(rng: int, v: int) -> int:
    return int(lib().oracle_unquant_color(rng, v))


def unquant_weight(rng: int, v: int) -> int:
    return int(lib().oracle_unquant_weight(rng, v))


def ise_bits(count: int, rng: int) -> int:
    return int(lib().oracle_ise_bits(count, rng))


def decode_trits(T: int):
    out = (ct.c_int * 5)()
    lib().oracle_decode_trits(T, out)
    return list(out)


def decode_quints(Q: int):
    out = (ct.c_int * 3)()
    lib().oracle_decode_quints(Q, out)
    return list(out)


LEVELS = (2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32, 40, 48, 64, 80, 96, 128, 160, 192, 256)


def read_astc_file(raw: bytes):
    """Parse the reference's .astc container (astc_kv/codec.py:110-113;
    metal/probe_gqa_v10.mm:116-134): magic, bx,by,bz, u24 w,h,d, payload."""
    if len(raw) < 16 or int.from_bytes(raw[:4], "little") != 0x5CA1AB13:
        raise ValueError("bad .astc magic")
    bx, by, bz = raw[4], raw[5], raw[6]
    w = int.from_bytes(raw[7:10], "little")
    h = int.from_bytes(raw[10:13], "little")
    d = int.from_bytes(raw[13:16], "little")
    return dict(bx=bx, by=by, bz=bz, width=w, height=h, depth=d, payload=raw[16:])
