"""Compact ASTC block atlas for a V cache (host side).

The reference keeps one .astc image per KV head and, for its GPU path, repacks
the 16-byte blocks of all heads into a 2D texture 32 blocks wide
(metal/probe_gqa_v10.mm:199-256). There is no texture sampler on gfx950, so the
atlas here is a plain linear array of blocks in exactly the reference's
staging order (head -> block row -> block column), with a sequence axis in
front: blocks[b, kv_head, row, col] is the block holding tokens
row*by .. row*by+by-1 and texel columns col*bx .. col*bx+bx-1 of that head's
image. Images follow astc_kv/codec.py's layouts (pack_images): scalar puts
channel c at texel x=c (R=G=B=u, A=1), rgba puts channels 4x..4x+3 in texel x.

V is token-normalised (codec.py:162-166): u = (v - o)/s with o = fp16_floor(min),
s = fp16_ceil(max - o), so V = u*s + o per token.
"""
from __future__ import annotations

import json
import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import codec


@dataclass
class Atlas:
    blocks: np.ndarray      # uint8 [B, Hkv, rows, cols, 16]
    scale: np.ndarray       # float16 [B, Hkv, T]
    offset: np.ndarray      # float16 [B, Hkv, T]
    tokens: int
    dim: int
    layout: str             # "scalar" | "rgba"
    block_x: int
    block_y: int
    page_tokens: int

    @property
    def batch(self) -> int:
        return self.blocks.shape[0]

    @property
    def kv_heads(self) -> int:
        return self.blocks.shape[1]

    @property
    def rows(self) -> int:
        return self.blocks.shape[2]

    @property
    def cols(self) -> int:
        return self.blocks.shape[3]

    def byte_counts(self) -> dict:
        """Persistent bytes of the compressed V: blocks (with padding) + fp16 metadata."""
        return {"astc_blocks": int(self.blocks.nbytes), "fp16_scales": int(self.scale.nbytes),
                "fp16_offsets": int(self.offset.nbytes)}

    def normalized(self) -> np.ndarray:
        """CPU decode of u [B, Hkv, T, D] (float32 holding FP16 values) via libakv_astc."""
        lib = codec.load_codec_library()
        flat = np.ascontiguousarray(self.blocks.reshape(-1, 16))
        tex = np.empty((flat.shape[0], self.block_y, self.block_x, 4), np.uint16)
        rc = lib.akv_decode_blocks_fp16(self.block_x, self.block_y, flat.ctypes.data, flat.shape[0],
                                        tex.ctypes.data, None)
        if rc:
            raise RuntimeError(lib.akv_error(rc).decode())
        b, h, r, c = self.blocks.shape[:4]
        img = tex.view(np.float16).reshape(b, h, r, c, self.block_y, self.block_x, 4)
        img = img.transpose(0, 1, 2, 4, 3, 5, 6).reshape(b, h, r * self.block_y, c * self.block_x, 4)
        img = img[:, :, : self.tokens].astype(np.float32)
        if self.layout == "scalar":
            return np.ascontiguousarray(img[..., : self.dim, 0])
        return np.ascontiguousarray(img[:, :, :, : self.dim // 4, :].reshape(b, h, self.tokens, self.dim))

    def restored(self) -> np.ndarray:
        """V = fl32(fl32(u*s) + o) [B, Hkv, T, D] (codec.py:206 order of operations)."""
        u = self.normalized()
        return u * self.scale.astype(np.float32)[..., None] + self.offset.astype(np.float32)[..., None]


def block_class_histogram(blocks: np.ndarray, block_x: int, block_y: int, layout: str) -> dict:
    """How the GPU decoder will treat an atlas's blocks (what its decode cost
    depends on): fractions of void-extent and error blocks, of blocks whose
    texels come from the per-block table (identity weight grid, one plane,
    partitions x weight levels <= 8 RGBA / 32 scalar entries) or are computed,
    of reduced weight grids and dual-plane blocks, and histograms of partition
    counts, weight levels and endpoint modes (libakv_astc akv_block_classes)."""
    lib = codec.load_codec_library()
    flat = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 16)
    n = flat.shape[0]
    cls = np.empty(n, np.uint32)
    rc = lib.akv_block_classes(block_x, block_y, flat.ctypes.data, n, cls.ctypes.data)
    if rc:
        raise RuntimeError(lib.akv_error(rc).decode())
    kind = cls & 3
    normal = kind == 0
    parts = ((cls >> 2) & 3) + 1
    dual = ((cls >> 4) & 1).astype(bool)
    identity = ((cls >> 5) & 1).astype(bool)
    levels = (cls >> 6) & 63
    cem = (cls >> 12) & 15
    entries = 32 if layout == "scalar" else 8
    table = normal & identity & ~dual & (parts * levels <= entries)

    def hist(values):
        v, c = np.unique(values[normal], return_counts=True)
        return {str(int(a)): round(float(b) / max(n, 1), 4) for a, b in zip(v, c)}

    frac = lambda m: round(float(np.count_nonzero(m)) / max(n, 1), 4)  # noqa: E731
    return {"blocks": int(n), "table_path": frac(table), "compute_path": frac(normal & ~table),
            "reduced_grid": frac(normal & ~identity), "dual_plane": frac(normal & dual),
            "void_extent": frac(kind == 1), "error": frac(kind == 2), "partitions": hist(parts),
            "weight_levels": hist(levels), "endpoint_modes": hist(cem)}


def texel_columns(dim: int, layout: str) -> int:
    return dim if layout == "scalar" else dim // 4


def normalize_tokens(v: np.ndarray):
    """Token range normalisation of [..., T, D] -> (u in [0,1], offset f16, scale f16)."""
    v = np.asarray(v, np.float32)
    offset = codec.fp16_floor(v.min(-1))
    spread = v.max(-1) - offset.astype(np.float32)
    scale = codec.fp16_ceil(np.maximum(spread, np.float32(2 ** -24)))
    u = (v - offset.astype(np.float32)[..., None]) / scale.astype(np.float32)[..., None]
    if u.min() < -1e-5 or u.max() > 1 + 1e-5:
        raise AssertionError("FP16 rounded metadata fails range coverage")
    return np.clip(u, 0, 1), offset, scale


def _encode_parallel(texels: np.ndarray, block_x: int, block_y: int, quality: float, threads: int) -> np.ndarray:
    n = texels.shape[0]
    out = np.empty((n, 16), np.uint8)
    threads = max(1, min(threads, n // 256 + 1))
    bounds = np.linspace(0, n, threads + 1).astype(int)

    def work(i):
        enc = codec.AstcEncoder((block_x, block_y), quality)
        try:
            out[bounds[i]:bounds[i + 1]] = enc.encode_blocks(texels[bounds[i]:bounds[i + 1]])
        finally:
            enc.close()

    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(work, range(threads)))
    return out


def build_atlas(v: np.ndarray, layout: str = "rgba", block=(6, 5), page_tokens: int = 120,
                quality: float = 50, threads: int | None = None) -> Atlas:
    """Token-normalise and ASTC-encode a V cache [B, Hkv, T, D] into an Atlas.

    Tokens are padded to a whole page by repeating the last token (the
    reference's fixture export pads the same way, scripts/export_metal_fixture.py:48);
    metadata is kept for the T real tokens only."""
    v = np.asarray(v, np.float32)
    if v.ndim != 4 or not np.isfinite(v).all():
        raise ValueError("Expected finite [B, Hkv, T, D]")
    bx, by = codec._footprint(block)
    b, h, t, d = v.shape
    if page_tokens % by:
        raise ValueError("page_tokens must be a multiple of the block height")
    if layout not in ("scalar", "rgba") or (layout == "rgba" and d % 4):
        raise ValueError("Unsupported layout")
    t_pad = codec.align(t, page_tokens)
    padded = np.pad(v, ((0, 0), (0, 0), (0, t_pad - t), (0, 0)), mode="edge")
    u, offset, scale = normalize_tokens(padded)
    width = codec.align(texel_columns(d, layout), bx)
    images = codec.pack_images(u.reshape(b * h, t_pad, d), layout, width)      # [B*H, T_pad, W, 4]
    rows, cols = t_pad // by, width // bx
    tiles = images.reshape(b * h, rows, by, cols, bx, 4).transpose(0, 1, 3, 2, 4, 5)
    tiles = np.ascontiguousarray(tiles.reshape(-1, by, bx, 4))
    blocks = _encode_parallel(tiles, bx, by, quality, threads or os.cpu_count() or 1)
    return Atlas(blocks.reshape(b, h, rows, cols, 16), np.ascontiguousarray(scale[:, :, :t]),
                 np.ascontiguousarray(offset[:, :, :t]), t, d, layout, bx, by, page_tokens)


def replicate_rows(atlas: Atlas, tokens: int) -> Atlas:
    """Longer context by repeating block rows and metadata along the token axis
    (the reference's traffic fixtures, scripts/make_traffic_fixture.py:12-49)."""
    if atlas.tokens % atlas.block_y:
        raise ValueError("source tokens must fill whole block rows")
    t_pad = codec.align(tokens, atlas.page_tokens)
    src_rows = atlas.tokens // atlas.block_y
    rows = np.arange(t_pad // atlas.block_y) % src_rows
    idx = np.arange(tokens) % atlas.tokens
    return Atlas(np.ascontiguousarray(atlas.blocks[:, :, rows]), np.ascontiguousarray(atlas.scale[:, :, idx]),
                 np.ascontiguousarray(atlas.offset[:, :, idx]), tokens, atlas.dim, atlas.layout, atlas.block_x,
                 atlas.block_y, atlas.page_tokens)


def read_astc(path: Path):
    raw = Path(path).read_bytes()
    if len(raw) < 16 or int.from_bytes(raw[:4], "little") != 0x5CA1AB13:
        raise ValueError(f"{path}: not an .astc file")
    bx, by, bz = raw[4], raw[5], raw[6]
    w, hgt = int.from_bytes(raw[7:10], "little"), int.from_bytes(raw[10:13], "little")
    if bz != 1:
        raise ValueError(f"{path}: 3D blocks are not supported")
    cols, rows = -(-w // bx), -(-hgt // by)
    payload = np.frombuffer(raw, np.uint8, count=rows * cols * 16, offset=16)
    if payload.size != rows * cols * 16:
        raise ValueError(f"{path}: truncated payload")
    return bx, by, w, hgt, payload.reshape(rows, cols, 16)


def atlas_from_manifest(directory: Path) -> tuple[Atlas, dict]:
    """Load the V side of an `astc-kv-probe-v1` fixture directory (reference
    interchange, docs/metal_path.md:50-73) as a batch-1 Atlas."""
    directory = Path(directory)
    m = json.loads((directory / "manifest.json").read_text())
    if m.get("format") != "astc-kv-probe-v1" or m.get("v_storage") != "astc":
        raise ValueError("expected an astc-kv-probe-v1 manifest with ASTC V")
    if m.get("v_normalization") != "token":
        raise ValueError("only token-normalised V is supported")
    t, h, d = m["tokens"], m["kv_heads"], m["head_dim"]
    heads = [read_astc(directory / f) for f in m["v_files"]]
    bx, by, w, hgt, _ = heads[0]
    if any(x[:4] != heads[0][:4] for x in heads) or hgt < t:
        raise ValueError("inconsistent .astc headers")
    layout = m.get("layout", "scalar")
    if w != codec.align(texel_columns(d, layout), bx):
        raise ValueError("atlas width does not match head_dim/layout")
    blocks = np.stack([x[4] for x in heads])[None]
    scale = np.fromfile(directory / m["v_scale_file"], "<f2").reshape(1, h, t)
    offset = np.fromfile(directory / m["v_offset_file"], "<f2").reshape(1, h, t)
    return Atlas(np.ascontiguousarray(blocks), scale, offset, t, d, layout, bx, by, m["page_tokens"]), m
